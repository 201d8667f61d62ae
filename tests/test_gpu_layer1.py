"""GPU parity of the one-launch decode layer (keep_moe_layer1): the router's
outputs equal the two-launch layer's (the same device code) bit for bit, the
layer output matches the C oracle (oracle/cpu_ref.c: LUT decode, fp32 sums, h
rounded to bf16) within 2e-3 elementwise, every served (I, k) tile shape and
both router lane widths run, the workspace's call counter advances once per
call, and a HIP graph of several layers replays to the eager outputs."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import nn as knn
from keep_amd import synth
from oracle import cpu, e8p, ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
OUT_TOL = {torch.float32: TOL, torch.bfloat16: TOL + 2.0 ** -9, torch.float16: TOL + 2.0 ** -11}


def _check(got, want, tol=TOL):
    g = got.float().cpu().numpy()
    err = ops.max_rel_err(g, want)
    assert err <= tol, f"max rel err {err:.3e}"
    assert ops.elementwise_ok(g, want, rtol=tol), "elementwise bound violated"
    assert not np.isnan(g).any()
    return err


def _oracle(x, r, gate, up, down, limit=0.0):
    """C-oracle output over the valid routes the layer served (an absent route
    carries weight 0 and no expert)."""
    idx = r.idx.cpu().numpy()
    w = r.weight.cpu().numpy().copy()
    ok = idx >= 0
    assert (w[~ok] == 0).all()
    used = np.unique(idx[ok])
    sub = {e: i for i, e in enumerate(used)}
    local = np.where(ok, np.vectorize(lambda e: sub.get(e, 0))(idx), 0).astype(np.int32)
    w[~ok] = 0.0
    sel = torch.from_numpy(used).to(gate.codes.device).long()
    pick = lambda p: (p.codes[sel].cpu().numpy().view(np.uint16), p.scales[sel].float().cpu().numpy())  # noqa: E731
    return cpu.moe_decode(x.float().cpu().numpy(), local, w, pick(gate), pick(up), pick(down),
                          e8p.e8p_packed_abs_grid(), limit=limit)


def _pool(E, I, gh, gi, seed):
    dev = torch.device("cuda", 0)
    return (synth.projection(E, I, 4096, group_size=gh, seed=seed, device=dev),
            synth.projection(E, I, 4096, group_size=gh, seed=seed + 1, device=dev),
            synth.projection(E, 4096, I, group_size=gi, seed=seed + 2, device=dev))


def _pairs(pool):
    return tuple((p.codes, p.scales) for p in pool)


def _workspace(dev, k, I):
    return torch.zeros(int(keep_amd._lib.load().keep_moe_layer1_workspace_bytes(k, I)), dtype=torch.uint8,
                       device=dev)


def _epoch(ws):
    return int(ws[:4].view(torch.int32).item())


def test_layer1_config2_vs_oracle_and_two_launch_router(dev):
    E, I, k = 384, 2048, 6
    pool = _pool(E, I, None, None, 1)
    x = synth.rht_activations(1, 4096, seed=4, device=dev)
    ws = _workspace(dev, k, I)
    for n, seed in enumerate((5, 6, 7)):
        print(f"layer1 config 2: logits seed {seed}", flush=True)
        z = synth.router_logits(1, E, seed=seed, device=dev)
        out, r = keep_amd.moe_layer(x, z, *_pairs(pool), k=k, one_launch=True, workspace=ws)
        two, r2 = keep_amd.moe_layer(x, z, *_pairs(pool), k=k)
        for a, b in zip(r, r2):
            assert torch.equal(a, b), "the one-launch router differs from the two-launch layer's"
        assert _epoch(ws) == n + 1 and knn.layer_status(ws) == 0
        _check(out, _oracle(x, r, *pool))
        _check(out, two.double().cpu().numpy())


# (E, I, k, group_h, group_i, x dtype, score func, SwiGLU limit, out dtype, resident fraction):
# every (tiles, slices, routes per wave) the dispatch serves, router lanes of 6 and 16 experts; k = 8 at
# I = 2048 (four q-tiles per block) is served by this layer only
CASES = [
    (288, 1536, 8, 1024, 512, torch.bfloat16, "softmax", 0.0, torch.float32, 0.5),
    (288, 1536, 6, 4096, 1536, torch.float16, "sigmoid", 7.0, torch.bfloat16, 1.0),
    (288, 1536, 5, 4096, 512, torch.float16, "softmax", 0.0, torch.float32, 1.0),
    (288, 1536, 4, 4096, 1536, torch.bfloat16, "sqrtsoftplus", 7.0, torch.float16, 1.0),  # limit: fp16 range
    (300, 1536, 2, 2048, 768, torch.float16, "softmax", 10.0, torch.float32, 1.0),
    (64, 1024, 3, 4096, 1024, torch.float16, "sqrtsoftplus", 0.0, torch.float32, 1.0),
    (64, 1024, 8, 512, 256, torch.bfloat16, "softmax", 0.0, torch.float32, 1.0),
    (40, 512, 8, 4096, 512, torch.float16, "sigmoid", 0.0, torch.float32, 1.0),
    (1024, 2048, 8, 4096, 2048, torch.bfloat16, "softmax", 0.0, torch.float32, 1.0),
    (500, 2048, 2, 4096, 2048, torch.float16, "softmax", 0.0, torch.float32, 0.25),
    (384, 2048, 4, 2048, 1024, torch.float16, "softmax", 0.0, torch.float32, 1.0),
]


@pytest.mark.parametrize("E,I,k,gh,gi,xdt,func,limit,odt,frac", CASES)
def test_layer1_served_shapes_vs_oracle(dev, E, I, k, gh, gi, xdt, func, limit, odt, frac):
    print(f"layer1: E={E} I={I} k={k} groups={gh}/{gi} x={xdt} {func} limit={limit} out={odt} resident={frac}",
          flush=True)
    pool = _pool(E, I, gh, gi, 11 + k)
    x = synth.rht_activations(1, 4096, seed=12, device=dev, dtype=xdt)
    z = synth.router_logits(1, E, seed=13, device=dev)
    bias = None
    if frac < 1.0:
        bias = keep_amd.resident_bias(torch.from_numpy(synth.resident_mask(E, frac=frac, seed=14)).to(dev))
    kw = dict(k=k, bias_served=bias, score_func=func, tau=0.3 if bias is not None else float("inf"), limit=limit,
              out_dtype=odt)
    ws = _workspace(dev, k, I)
    out, r = keep_amd.moe_layer(x, z, *_pairs(pool), one_launch=True, workspace=ws, **kw)
    ref = keep_amd.router_dual_topk(z, k, bias_served=bias, score_func=func, tau=kw["tau"])
    for a, b in zip(r, ref):
        assert torch.equal(a, b), "the one-launch router differs from the standalone router"
    assert out.dtype == odt and knn.layer_status(ws) == 0 and _epoch(ws) == 1
    _check(out, _oracle(x, r, *pool, limit=limit), OUT_TOL[odt])


def test_layer1_fewer_residents_than_k(dev):
    """Three resident experts under top-6: the other three routes name absent
    experts (the lowest ids, as the router's ordering of equal keys gives) with
    weight 0, and add nothing."""
    E, I, k = 384, 2048, 6
    pool = _pool(E, I, None, None, 21)
    mask = np.zeros(E, bool)
    mask[[7, 200, 383]] = True
    bias = keep_amd.resident_bias(torch.from_numpy(mask).to(dev))
    x = synth.rht_activations(1, 4096, seed=22, device=dev)
    z = synth.router_logits(1, E, seed=23, device=dev)
    out, r = keep_amd.moe_layer(x, z, *_pairs(pool), k=k, bias_served=bias, one_launch=True,
                                workspace=_workspace(dev, k, I))
    idx, w = r.idx.cpu().numpy()[0], r.weight.cpu().numpy()[0]
    assert sorted(idx[w > 0].tolist()) == [7, 200, 383] and (w == 0).sum() == 3
    _check(out, _oracle(x, r, *pool))


@pytest.mark.parametrize("place", [0, 5])
def test_layer1_early_route_tie_reloads(dev, place):
    """The tiles' loads issue on routes picked from the logits; they are used
    unchecked only when each selected logit is at least 2^-16 above the next.
    Here two logits differ by FLT_MIN (0 at expert 40, FLT_MIN at expert 300):
    both softmax scores are exp(0) / sum exactly, so the exact selection takes
    the lower index (40) and the logit order the higher (300). At place 0
    every block's first route differs; at place 5 (the sixth route) only the
    blocks holding tiles of route 5 do. Those blocks must reload their tiles:
    the router outputs equal the standalone router's, the output the oracle's,
    and no certified route differed (status 0)."""
    E, I, k = 384, 2048, 6
    pool = _pool(E, I, None, None, 51)
    x = synth.rht_activations(1, 4096, seed=52, device=dev)
    rng = np.random.default_rng(53)
    z = -1.0 - rng.random(E).astype(np.float32)  # every other logit below -1
    top = rng.choice([e for e in range(E) if e not in (40, 300)], size=place, replace=False)
    z[top] = np.float32(3.0) - np.arange(place, dtype=np.float32) * np.float32(0.5)
    z[40] = np.float32(0.0)
    z[300] = np.finfo(np.float32).tiny
    zt = torch.from_numpy(z.reshape(1, E)).to(dev)
    ref = keep_amd.router_dual_topk(zt, k)
    idx = ref.idx.cpu().numpy()[0]
    assert idx[place] == 40 and (place + 1 >= k or idx[place + 1] == 300), \
        "the exact selection breaks the score tie by index"
    ws = _workspace(dev, k, I)
    out, r = keep_amd.moe_layer(x, zt, *_pairs(pool), k=k, one_launch=True, workspace=ws)
    for a, b in zip(r, ref):
        assert torch.equal(a, b), "the one-launch router differs from the standalone router"
    assert knn.layer_status(ws) == 0
    _check(out, _oracle(x, r, *pool))
    two, _ = keep_amd.moe_layer(x, zt, *_pairs(pool), k=k)
    _check(out, two.double().cpu().numpy())


def test_layer1_finite_biases(dev):
    """Served biases that are neither 0 nor the residency mask (a score
    correction bias beside it): the tile routes come from the exact keys, and
    the outputs equal the standalone router's and the oracle's."""
    E, I, k = 384, 2048, 6
    pool = _pool(E, I, None, None, 61)
    x = synth.rht_activations(1, 4096, seed=62, device=dev)
    z = synth.router_logits(1, E, seed=63, device=dev)
    corr = torch.from_numpy(np.random.default_rng(64).normal(0.0, 0.05, E).astype(np.float32)).to(dev)
    mask = torch.from_numpy(synth.resident_mask(E, frac=0.5, seed=65)).to(dev)
    for bias in (corr, keep_amd.resident_bias(mask, corr)):
        ws = _workspace(dev, k, I)
        out, r = keep_amd.moe_layer(x, z, *_pairs(pool), k=k, bias_served=bias, one_launch=True, workspace=ws)
        ref = keep_amd.router_dual_topk(z, k, bias_served=bias)
        for a, b in zip(r, ref):
            assert torch.equal(a, b), "the one-launch router differs from the standalone router"
        assert knn.layer_status(ws) == 0
        _check(out, _oracle(x, r, *pool))


def test_layer1_graph_replays_match_eager(dev):
    """Four layers captured in one graph on a side stream (the workspace of that
    stream); three replays with eager work between them, each equal to the
    eager outputs bit for bit, and the call counter advanced by 4 per replay."""
    E, I, k, n = 384, 2048, 6, 4
    pool = _pool(E, I, None, None, 1)
    x = synth.rht_activations(1, 4096, seed=31, device=dev)
    zs = synth.router_logits(n, E, seed=32, device=dev).reshape(n, 1, E).contiguous()
    eager = [keep_amd.moe_layer(x, zs[i], *_pairs(pool), k=k, one_launch=True, workspace=_workspace(dev, k, I))[0]
             for i in range(n)]
    ws = _workspace(dev, k, I)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for i in range(n):  # warm-up outside the capture
            keep_amd.moe_layer(x, zs[i], *_pairs(pool), k=k, one_launch=True, workspace=ws)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            outs = [keep_amd.moe_layer(x, zs[i], *_pairs(pool), k=k, one_launch=True, workspace=ws)[0]
                    for i in range(n)]
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    base = _epoch(ws)
    assert base == n
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        for i in range(n):
            assert torch.equal(outs[i], eager[i]), f"replay {rep} layer {i} differs from eager"
        assert _epoch(ws) == base + n * (rep + 1) and knn.layer_status(ws) == 0
        keep_amd.moe_layer(x, zs[rep], *_pairs(pool), k=k, one_launch=True, workspace=_workspace(dev, k, I))
        torch.cuda.synchronize()


def test_layer1_give_up_path_and_recovery(dev):
    """A host-set spin budget of 0 ticks: a wave whose first poll finds another
    block's h not yet written gives up at once (every wait ends), writes NaN
    for the routes it holds and sets status bit 1; the router's outputs and
    every finite output equal a normal call's. With the default budget back
    and the workspace zeroed, the next call equals the normal call bit for bit."""
    E, I, k = 384, 2048, 6
    pool = _pool(E, I, None, None, 41)
    x = synth.rht_activations(1, 4096, seed=42, device=dev)
    z = synth.router_logits(1, E, seed=43, device=dev)
    ref, r_ref = keep_amd.moe_layer(x, z, *_pairs(pool), k=k, one_launch=True, workspace=_workspace(dev, k, I))
    ws = _workspace(dev, k, I)
    gave_up = False
    prev = knn.layer_spin_ticks(0)
    try:
        for attempt in range(3):
            print(f"layer1 give-up: budget 0, call {attempt}", flush=True)
            out, r = keep_amd.moe_layer(x, z, *_pairs(pool), k=k, one_launch=True, workspace=ws)
            torch.cuda.synchronize()
            for a, b in zip(r, r_ref):
                assert torch.equal(a, b)
            nan = torch.isnan(out)
            status = knn.layer_status(ws)
            assert bool(nan.any()) == bool(status & 1), "NaN outputs exactly when a wait gave up"
            assert torch.equal(out[~nan], ref[~nan])
            if status & 1:
                gave_up = True
                break
    finally:
        assert knn.layer_spin_ticks(prev) == 0
    assert prev == 20000 and gave_up, "no wait gave up under a budget of 0 ticks"
    ws.zero_()
    out, r = keep_amd.moe_layer(x, z, *_pairs(pool), k=k, one_launch=True, workspace=ws)
    assert knn.layer_status(ws) == 0 and torch.equal(out, ref)
    with pytest.raises(ValueError, match="spin budget"):
        knn.layer_spin_ticks(100000001)


def test_layer1_rejects_unserved(dev):
    E, I, k = 384, 2048, 6
    pool = _pool(E, I, None, None, 1)
    x = synth.rht_activations(1, 4096, seed=4, device=dev)
    z = synth.router_logits(1, E, seed=5, device=dev)
    with pytest.raises(ValueError, match="workspace"):
        keep_amd.moe_layer(x, z, *_pairs(pool), k=k, one_launch=True, workspace=_workspace(dev, k, 1024))
    with pytest.raises(ValueError, match="one-launch"):  # fewer than k experts
        keep_amd.moe_layer(x, z[:, :4], *_pairs(pool), k=k, one_launch=True, slot_map=torch.zeros(4, dtype=torch.int32,
                                                                                               device=dev))
