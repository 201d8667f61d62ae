"""GPU parity of the expert-grouped few-token MoE (keep_moe_tiles): byte
identity with the one-token layer token by token (the verify-rows discipline
of the reference, tests/test_gather_vqmm_verify_rows.py:1-33), the C oracle at
the verify shapes of config 3, the float64 oracle with many routes per expert
(several tiles and route chunks per expert), the combine's edge cases, and the
layer from the logits (keep_moe_tiles_layer: the gate/up launch routing and
planning itself up to 128 routes, or router, terms and plan in one prologue
launch up to 32 tokens) byte-identical to the router followed by the tiles."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import synth
from oracle import cpu, e8p, ops

pytestmark = pytest.mark.gpu
TOL = 2e-3


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


@pytest.fixture(scope="module")
def pool(dev):
    E, H, I = 384, 4096, 2048
    return (synth.projection(E, I, H, seed=1, device=dev), synth.projection(E, I, H, seed=2, device=dev),
            synth.projection(E, H, I, seed=3, device=dev))


def _pairs(pool):
    return tuple((p.codes, p.scales) for p in pool)


def test_tiles_byte_identical_to_one_token_layer(dev, pool):
    """Each token's output equals keep_moe_layer's for that token bit for bit."""
    E, H, I, k, T = 384, 4096, 2048, 6, 8
    assert keep_amd.nn.moe_tiles_supported(T, E, H, I, k, H, I)
    x = synth.rht_activations(T, H, seed=21, device=dev)
    z = synth.router_logits(T, E, seed=22, device=dev)
    z[1] = z[0]  # two tokens routed to the same experts: their routes share tiles
    r = keep_amd.router_dual_topk(z, k)
    out = keep_amd.moe_decode(x, r.idx, r.weight, *_pairs(pool))
    for t in range(T):
        one, rt = keep_amd.moe_layer(x[t:t + 1], z[t:t + 1], *_pairs(pool), k=k)
        assert torch.equal(rt.idx[0], r.idx[t])
        assert torch.equal(one[0], out[t]), f"token {t} differs from the one-token layer"


@pytest.mark.parametrize("T", [16, 64])
def test_tiles_verify_shapes_vs_c_oracle(dev, pool, T):
    E, H, I, k = 384, 4096, 2048, 6
    x = synth.rht_activations(T, H, seed=30 + T, device=dev)
    z = synth.router_logits(T, E, seed=40 + T, device=dev)
    r = keep_amd.router_dual_topk(z, k)
    out = keep_amd.moe_decode(x, r.idx, r.weight, *_pairs(pool))
    idx = r.idx.cpu().numpy()
    used = np.unique(idx)
    sub = {e: i for i, e in enumerate(used)}
    sel = torch.from_numpy(used).to(dev).long()
    pick = lambda p: (p.codes[sel].cpu().numpy().view(np.uint16), p.scales[sel].float().cpu().numpy())  # noqa: E731
    local = np.vectorize(sub.get)(idx).astype(np.int32)
    want = cpu.moe_decode(x.float().cpu().numpy(), local, r.weight.cpu().numpy(), *(pick(p) for p in pool),
                          e8p.e8p_packed_abs_grid())
    _check(out, want)


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_tiles_many_routes_per_expert_vs_oracle(dev, xdt):
    """Four experts, 48 tokens x 3 routes: ~36 routes per expert, so several
    16-route tiles per expert and several A chunks per tile."""
    E, H, I, k, T = 4, 512, 512, 3, 48
    gate = synth.projection_np(E, I, H, group_size=256, seed=51)
    up = synth.projection_np(E, I, H, group_size=256, seed=52)
    down = synth.projection_np(E, H, I, seed=53)
    x = synth.rht_activations(T, H, seed=54, device=dev, dtype=xdt)
    z = synth.router_logits(T, E, seed=55, device=dev)
    r = keep_amd.router_dual_topk(z, k)
    counts = np.bincount(r.idx.cpu().numpy().ravel(), minlength=E)
    assert counts.max() > 16
    tt = lambda p: (_t(p[0], dev), _t(p[1], dev))  # noqa: E731
    out = keep_amd.moe_decode(x, r.idx, r.weight, tt(gate), tt(up), tt(down), limit=7.0)
    want = ops.moe_layer(x.float().cpu().numpy(), r.idx.cpu().numpy(), r.weight.cpu().numpy(), gate, up, down,
                         limit=7.0, h_round="bfloat16")
    _check(out, want)


def test_tiles_blocks_across_three_tiles_vs_oracle(dev):
    """256 tokens x 8 routes over 16 experts (512 tiles of 4 routes): a gate/up block takes 32 units of
    16-unit tiles and a down block 8 units of 4-unit tiles, so blocks start mid-tile and run through up to
    three tiles, their code loads crossing each tile boundary two units ahead.

    Each stage is checked on its own: every stored h (bf16, the route's row of h_work) lies within one bf16
    ulp of the float64 SwiGLU (plus 1e-4 of the row's rms where the dots cancel), and the output lies within
    the bound of the down kernel's arithmetic around the float64 down and combine of the stored h: each h
    element enters as two int8 terms under a power of two per 256-wide slice, 2^(e - 6) with
    2^(e - 1) <= max |h| < 2^e, so it is off by at most 2^(e - 14); the rest is exact int32 sums and fp32
    scaling. With I = 256 and one heavy-tailed slice per route, an end-to-end bound against the float64
    layer would measure bf16 ties and that split, not the schedule."""
    E, H, I, k, T = 16, 256, 256, 8, 256
    gate = synth.projection_np(E, I, H, seed=71)
    up = synth.projection_np(E, I, H, seed=72)
    down = synth.projection_np(E, H, I, seed=73)
    x = synth.rht_activations(T, H, seed=74, device=dev)
    z = synth.router_logits(T, E, seed=75, device=dev)
    r = keep_amd.router_dual_topk(z, k)
    assert keep_amd.nn.moe_tiles_supported(T, E, H, I, k, H, I)
    tt = lambda p: (_t(p[0], dev), _t(p[1], dev))  # noqa: E731
    h_work = torch.empty((T * k * I,), dtype=torch.bfloat16, device=dev)
    out = keep_amd.moe_decode(x, r.idx, r.weight, tt(gate), tt(up), tt(down), h_work=h_work)
    h = h_work.float().cpu().numpy().reshape(T, k, I).astype(np.float64)
    xs = x.float().cpu().numpy().astype(np.float64)
    idx, w = r.idx.cpu().numpy(), r.weight.cpu().numpy().astype(np.float64)
    wg, wu, wd = ops.dense(*gate), ops.dense(*up), ops.dense(*down)
    want, bound = np.zeros((T, H)), np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            e = idx[t, j]
            h64 = ops.swiglu(wg[e] @ xs[t], wu[e] @ xs[t])
            ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(h64), 2.0 ** -126))) - 7)
            hb = ulp + 1e-4 * np.sqrt(np.mean(h64 * h64))
            assert np.all(np.abs(h[t, j] - h64) <= hb), f"h of token {t} route {j} (expert {e})"
            want[t] += w[t, j] * (wd[e] @ h[t, j])
            mx = np.abs(h[t, j]).reshape(-1, 256).max(axis=1)
            step = np.where(mx > 0, 2.0 ** (np.floor(np.log2(np.maximum(mx, 2.0 ** -126))) + 1 - 14), 0.0)
            bound[t] += abs(w[t, j]) * (np.abs(wd[e]) @ (np.repeat(step, 256) + 1e-6 * np.abs(h[t, j])))
    g = out.float().cpu().numpy()
    assert ops.max_rel_err(g, want) <= TOL
    assert np.all(np.abs(g - want) <= bound), f"worst excess {np.max(np.abs(g - want) - bound):.3g}"


def test_tiles_zero_weight_and_bad_expert(dev):
    """A zero-weight route adds nothing; an out-of-range expert with a weight
    makes its token's row NaN and leaves the others intact."""
    E, H, I, k, T = 8, 256, 256, 2, 3
    gate = synth.projection_np(E, I, H, seed=61)
    up = synth.projection_np(E, I, H, seed=62)
    down = synth.projection_np(E, H, I, seed=63)
    x = synth.rht_activations(T, H, seed=64, device=dev)
    idx = torch.tensor([[1, 2], [3, 99], [5, -4]], dtype=torch.int32, device=dev)
    w = torch.tensor([[0.7, 0.0], [0.4, 0.6], [1.0, 0.0]], dtype=torch.float32, device=dev)
    tt = lambda p: (_t(p[0], dev), _t(p[1], dev))  # noqa: E731
    out = keep_amd.moe_decode(x, idx, w, tt(gate), tt(up), tt(down)).cpu()
    assert torch.isnan(out[1]).all()
    good = np.array([[1, 2], [5, 0]], dtype=np.int32)
    gw = np.array([[0.7, 0.0], [1.0, 0.0]], dtype=np.float32)
    want = ops.moe_layer(x[[0, 2]].float().cpu().numpy(), good, gw, gate, up, down, h_round="bfloat16")
    _check(out[[0, 2]], want)


@pytest.fixture(scope="module")
def small_pool(dev):
    E, H, I = 1000, 1024, 512
    return (synth.projection(E, I, H, seed=5, device=dev), synth.projection(E, I, H, seed=6, device=dev),
            synth.projection(E, H, I, seed=7, device=dev))


@pytest.mark.parametrize("T, E, xdt, biased", [(2, 384, torch.float16, False), (8, 384, torch.float16, False),
                                              (16, 100, torch.bfloat16, True), (20, 384, torch.bfloat16, False),
                                              (21, 500, torch.float16, True), (22, 384, torch.float16, False),
                                              (32, 1000, torch.float16, True), (33, 384, torch.float16, False),
                                              (64, 300, torch.bfloat16, True), (65, 384, torch.float16, False)])
def test_tiles_layer_equals_router_then_tiles(dev, small_pool, T, E, xdt, biased):
    """keep_moe_tiles_layer: the router's five outputs and the tiles' result, bit for bit, on every side of
    its launch forms: routed gate/up (up to 128 routes and 512 experts; 20 and 21 tokens put two tokens on
    some routing waves), the prologue (22 and 32 tokens), the router launch (33 and more); every router
    lane width, with and without biases and admission."""
    from keep_amd.router import resident_bias
    H, I, k = 1024, 512, 6
    pool = tuple((p.codes[:E], p.scales[:E]) for p in small_pool)
    x = synth.rht_activations(T, H, seed=60 + T, device=dev).to(xdt)
    z = synth.router_logits(T, E, seed=61 + T, device=dev)
    kw = {}
    if biased:
        mask = torch.from_numpy(synth.resident_mask(E, frac=0.5, seed=62)).to(dev)
        kw = dict(bias_served=resident_bias(mask), bias_demand=None, tau=0.3)
    r = keep_amd.router_dual_topk(z, k, **kw)
    want = keep_amd.moe_decode(x, r.idx, r.weight, *pool)
    out, r2 = keep_amd.moe_tiles_layer(x, z, *pool, k=k, **kw)
    for name in ("idx", "weight", "want", "want_score", "admit"):
        assert torch.equal(getattr(r2, name), getattr(r, name)), f"router output {name} differs"
    assert torch.equal(out, want), "layer output differs from the router followed by keep_moe_tiles"


def test_tiles_layer_slot_map_and_module(dev, small_pool):
    """A pool of 256 rows under a 1000-expert router (slot map), and RoutedVQMoE's few-token call."""
    E, S, H, I, k, T = 1000, 256, 1024, 512, 6, 8
    pool = tuple((p.codes[:S], p.scales[:S]) for p in small_pool)
    rng = np.random.default_rng(70)
    sm_np = np.full(E, -1, dtype=np.int32)
    sm_np[rng.choice(E, S, replace=False)] = np.arange(S, dtype=np.int32)
    sm = torch.from_numpy(sm_np).to(dev)
    from keep_amd.router import resident_bias
    bias = resident_bias(sm >= 0)
    x = synth.rht_activations(T, H, seed=71, device=dev)
    z = synth.router_logits(T, E, seed=72, device=dev)
    r = keep_amd.router_dual_topk(z, k, bias_served=bias, slot_map=sm, num_slots=S)
    want = keep_amd.moe_decode(x, r.idx, r.weight, *pool)
    out, r2 = keep_amd.moe_tiles_layer(x, z, *pool, k=k, bias_served=bias, slot_map=sm)
    assert torch.equal(r2.idx, r.idx) and torch.equal(r2.weight, r.weight)
    assert torch.equal(out, want)
    lin = lambda p, i, o: keep_amd.QuantizedVQSwitchLinear(  # noqa: E731
        input_dims=i, output_dims=o, num_experts=S, codes=p.codes[:S], scales=p.scales[:S], group_size=i,
        code_bits=16)
    g, u, d = small_pool
    moe = keep_amd.RoutedVQMoE(keep_amd.QuantizedVQSwitchGLU(gate_proj=lin(g, H, I), up_proj=lin(u, H, I),
                                                             down_proj=lin(d, I, H)),
                               top_k=k, bias_served=bias, slot_map=sm)
    out_m, r_m = moe(x, z)
    assert torch.equal(r_m.idx, r.idx) and torch.equal(out_m, want)


@pytest.mark.parametrize("T", [8, 16])
def test_tiles_layer_config3_shape(dev, pool, T):
    """Config 3's shape (384 experts, 4096 / 2048, top-6) from the logits, routed gate/up: every K slice
    forms its own terms, blocks cross tiles; bit for bit with the router followed by keep_moe_tiles."""
    E, H, I, k = 384, 4096, 2048, 6
    x = synth.rht_activations(T, H, seed=80 + T, device=dev)
    z = synth.router_logits(T, E, seed=81 + T, device=dev)
    z[3] = z[2]  # two tokens on the same experts: tiles of two routes
    r = keep_amd.router_dual_topk(z, k)
    want = keep_amd.moe_decode(x, r.idx, r.weight, *_pairs(pool))
    out, r2 = keep_amd.moe_tiles_layer(x, z, *_pairs(pool), k=k)
    assert torch.equal(r2.idx, r.idx) and torch.equal(r2.weight, r.weight)
    assert torch.equal(out, want)


def test_tiles_layer_absent_experts(dev, small_pool):
    """A slot map without the residency bias: some selected experts have no pool row (slot -1), their
    routes sort last and are not computed, and their tokens' outputs are NaN, exactly as the router
    followed by keep_moe_tiles gives them (routed gate/up, 400 experts over 200 rows)."""
    E, S, H, I, k, T = 400, 200, 1024, 512, 6, 12
    pool = tuple((p.codes[:S], p.scales[:S]) for p in small_pool)
    rng = np.random.default_rng(90)
    sm_np = np.full(E, -1, dtype=np.int32)
    sm_np[rng.choice(E, S, replace=False)] = np.arange(S, dtype=np.int32)
    sm = torch.from_numpy(sm_np).to(dev)
    x = synth.rht_activations(T, H, seed=91, device=dev)
    z = synth.router_logits(T, E, seed=92, device=dev)
    r = keep_amd.router_dual_topk(z, k, slot_map=sm, num_slots=S)
    assert (r.idx < 0).any() and (r.idx >= 0).any()
    want = keep_amd.moe_decode(x, r.idx, r.weight, *pool)
    out, r2 = keep_amd.moe_tiles_layer(x, z, *pool, k=k, slot_map=sm)
    assert torch.equal(r2.idx, r.idx) and torch.equal(r2.weight, r.weight)
    nan = torch.isnan(want)
    assert nan.any() and torch.equal(torch.isnan(out), nan)
    assert torch.equal(out[~nan], want[~nan])


def test_tiles_layer_near_ties_fall_back_to_exact_keys(dev, small_pool):
    """Routed gate/up: its blocks select on the logits where the softmax certifies that order. Tokens whose
    logits differ by one ulp with equal softmax scores (the larger logit on the higher index, so the logit
    order and the score order disagree), at the first route, at the last route against the first left out,
    and twice among the routes: the layer still equals the router followed by keep_moe_tiles bit for bit."""
    E, H, I, k, T = 384, 1024, 512, 6, 8
    pool = tuple((p.codes[:E], p.scales[:E]) for p in small_pool)
    x = synth.rht_activations(T, H, seed=95, device=dev)
    z = synth.router_logits(T, E, seed=96, device=dev) - 8.0
    up1 = lambda v: float(np.nextafter(np.float32(v), np.float32(np.inf)))  # noqa: E731
    z[0, 40], z[0, 300] = 0.0, float(np.finfo(np.float32).tiny)       # the first route
    for j, e in enumerate((10, 11, 12, 13, 14)):                       # routes 0-4, then the sixth
        z[1, e] = 5.0 - j
    z[1, 100], z[1, 200] = 0.5, up1(0.5)
    z[2, 9] = 5.0                                                      # two pairs among the routes
    z[2, 7], z[2, 300] = 0.25, up1(0.25)
    z[2, 8], z[2, 301] = 0.125, up1(0.125)
    z[3, 40], z[3, 41] = 3.0, 3.0                                      # an exact tie
    r = keep_amd.router_dual_topk(z, k)
    # the cases bite: the score order puts the lower index first where the logit order would not
    assert r.idx[0, 0].item() == 40 and r.idx[1, 5].item() == 100
    assert r.idx[2, 1].item() == 7 and r.idx[2, 3].item() == 8
    want = keep_amd.moe_decode(x, r.idx, r.weight, *pool)
    out, r2 = keep_amd.moe_tiles_layer(x, z, *pool, k=k)
    assert torch.equal(r2.idx, r.idx) and torch.equal(r2.weight, r.weight)
    assert torch.equal(out, want)
