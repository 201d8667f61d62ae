"""A pool smaller than the expert count on the GPU: a ResidencyCache of 8 slots
over a 32-expert layer file, the no-wait policy driving installs through
ExpertInstaller while the fused decode layer serves from the slots.

Every call: the served routing equals the oracle router's top-k over the
experts resident at that call (OFF bias for the others) with the router's
outputs naming pool rows (slot_map), and the layer output matches the C
oracle run on those experts' codes read from the file. Strongly demanded
absent experts are read in and routed only after their copies land (then
served); the pool rows hold the file's bytes of their experts throughout."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import loaders, synth
from keep_amd.residency import ROUTED, ResidencyCache, ResidencyPolicy
from oracle import cpu, e8p, ops

pytestmark = pytest.mark.gpu
E, S, H, I, K = 32, 8, 4096, 512, 4


def _write_layer(path):
    arrays = {}
    for proj, (n, k), seed in (("w1", (I, H), 1), ("w3", (I, H), 2), ("w2", (H, I), 3)):
        codes, scales = synth.projection_np(E, n, k, seed=seed)
        arrays[f"{proj}_codes"], arrays[f"{proj}_scales"] = codes, scales
    np.savez(path, code_bits=np.asarray(16), **arrays)
    return arrays


def _pools(dev):
    def pair(n, k):
        return (torch.zeros((S, n, k // 8), dtype=torch.int16, device=dev),
                torch.zeros((S, n, 1), dtype=torch.float16, device=dev))
    return {"w1": pair(I, H), "w3": pair(I, H), "w2": pair(H, I)}


@pytest.mark.parametrize("one_launch", [False, True])
def test_pool_smaller_than_experts_serves_residents_and_installs(dev, tmp_path, one_launch):
    print(f"residency: E={E} slots={S} one_launch={one_launch}", flush=True)
    arrays = _write_layer(tmp_path / "layer-00.npz")
    layer = loaders.LayerFile(tmp_path / "layer-00.npz")
    pools = _pools(dev)
    inst = loaders.ExpertInstaller(layer, pools, dev)
    order = list(range(E))  # experts 0..7 start resident
    cache = ResidencyCache(inst, E, order, tau=0.2, spare=1, lag=1)
    x = synth.rht_activations(1, H, seed=5, device=dev)
    rng = np.random.default_rng(6)
    tab = e8p.e8p_packed_abs_grid()
    host = {p: (arrays[f"{p}_codes"], arrays[f"{p}_scales"].astype(np.float32)) for p in ("w1", "w3", "w2")}
    hot = [20, 27]  # demanded strongly every call: absent at first
    served_hot = False
    for step in range(12):
        cache.begin()
        torch.cuda.synchronize()
        slot_expert = cache.table().slot_expert()
        resident = cache.resident_mask()
        for s, e in enumerate(slot_expert):  # every routed row holds its expert's file bytes
            if e >= 0:
                np.testing.assert_array_equal(pools["w1"][0][s].cpu().numpy().view(np.uint16), arrays["w1_codes"][e])
                np.testing.assert_array_equal(pools["w2"][0][s].cpu().numpy().view(np.uint16), arrays["w2_codes"][e])
        z_np = rng.standard_normal((1, E)).astype(np.float32)
        z_np[0, hot] += 6.0
        z = torch.from_numpy(z_np).to(dev)
        out, r = keep_amd.moe_layer(x, z, pools["w1"], pools["w3"], pools["w2"], k=K,
                                    bias_served=cache.bias(), tau=cache.tau, slot_map=cache.slots(),
                                    one_launch=one_launch,
                                    workspace=None if not one_launch else keep_amd.nn.layer_workspace(dev, K, I))
        cache.observe(r)
        # the router: top-k over the residents, outputs as pool rows
        bias = np.where(resident, 0.0, ops.MASKED_BIAS)
        oi, ow, owant, _, _ = ops.router_dual_topk(z_np, bias, np.zeros(E), K, tau=cache.tau)
        slot_of = {int(e): s for s, e in enumerate(slot_expert) if e >= 0}
        want_rows = np.array([[slot_of.get(int(e), -1) for e in oi[0]]])
        live = ow > 0
        np.testing.assert_array_equal(r.idx.cpu().numpy()[live], want_rows[live])
        np.testing.assert_allclose(r.weight.cpu().numpy(), ow, rtol=1e-5, atol=1e-7)
        np.testing.assert_array_equal(r.want.cpu().numpy(), owant)  # demand: expert ids over the whole pool
        experts = oi[0][live[0]]
        assert resident[experts].all()
        served_hot |= bool(np.isin(hot, experts).any())
        # the output: the C oracle on the served experts' file codes
        used = np.unique(experts)
        local = np.searchsorted(used, experts).astype(np.int32)[None]
        pick = lambda p: (host[p][0][used], host[p][1][used])  # noqa: E731
        want = cpu.moe_decode(x.float().cpu().numpy(), local, ow[live][None], pick("w1"), pick("w3"), pick("w2"), tab)
        err = ops.max_rel_err(out.cpu().numpy(), want)
        assert err <= 2e-3, f"step {step}: max rel err {err:.3e}"
    assert cache.stats["installed"] >= 2 and cache.stats["evicted"] >= 2
    assert all(h in cache.table().assignment() for h in hot), "strongly demanded experts are resident by now"
    assert cache.mismatched() == 0
    assert served_hot, "an installed expert was served"


def test_route_only_after_copy_event(dev, tmp_path):
    """The policy routes an expert only once installer.ready(event) holds: a
    read that has not landed keeps the expert unrouted across harvests."""
    _write_layer(tmp_path / "layer-00.npz")
    layer = loaders.LayerFile(tmp_path / "layer-00.npz")
    pools = _pools(dev)
    inst = loaders.ExpertInstaller(layer, pools, dev)

    class Held(ResidencyCache):
        hold = True

        def done(self, handle):
            return (not self.hold) and super().done(handle)

    cache = Held(inst, E, list(range(E)), tau=0.2, spare=1, lag=1)
    want = np.array([[30, 0, 1, 2]], np.int32)
    score = np.array([[5.0, 0.1, 0.1, 0.1]], np.float32)
    for _ in range(4):
        cache.begin()
        ResidencyPolicy.observe(cache, want, score)  # host demand, as a finished call's
    assert cache.table().read_at[30] >= 0 and 30 not in cache.table().assignment()
    assert cache.bias()[30].item() <= ops.MASKED_BIAS
    cache.hold = False
    torch.cuda.synchronize()
    cache.begin()
    torch.cuda.synchronize()
    slot = cache.table().assignment()[30]
    assert cache.bias()[30].item() == 0.0 and cache.slots()[30].item() == slot
    np.testing.assert_array_equal(pools["w3"][0][slot].cpu().numpy().view(np.uint16), layer.read("w3_codes", [30])[0])


@pytest.mark.parametrize("T", [1, 5, 96])
def test_routed_moe_over_slots_all_paths(dev, tmp_path, T):
    """RoutedVQMoE over an 8-row pool with the cache's slot map and served
    bias: the fused layer (T = 1), the few-token kernels (T = 5) and the
    prefill grouped GEMMs (T = 96) all read each served expert at its row."""
    arrays = _write_layer(tmp_path / "layer-00.npz")
    layer = loaders.LayerFile(tmp_path / "layer-00.npz")
    pools = _pools(dev)
    order = [3, 17, 8, 30, 1, 12, 25, 6] + [e for e in range(E) if e not in (3, 17, 8, 30, 1, 12, 25, 6)]
    cache = ResidencyCache(loaders.ExpertInstaller(layer, pools, dev), E, order, tau=0.2, spare=1, lag=1)

    def lin(p, K, N):
        return keep_amd.QuantizedVQSwitchLinear(input_dims=K, output_dims=N, num_experts=S, codes=pools[p][0],
                                                scales=pools[p][1], group_size=K, code_bits=16)
    glu = keep_amd.QuantizedVQSwitchGLU(gate_proj=lin("w1", H, I), up_proj=lin("w3", H, I),
                                        down_proj=lin("w2", I, H))
    moe = keep_amd.RoutedVQMoE(glu, top_k=K, bias_served=cache.bias(), slot_map=cache.slots())
    x = synth.rht_activations(T, H, seed=T, device=dev)
    z = synth.router_logits(T, E, seed=T + 1, device=dev)
    out, r = moe(x, z)
    bias = np.where(cache.resident_mask(), 0.0, ops.MASKED_BIAS)
    oi, ow, *_ = ops.router_dual_topk(z.cpu().numpy(), bias, np.zeros(E), K)
    np.testing.assert_array_equal(r.idx.cpu().numpy(), np.vectorize(cache.table().assignment().get)(oi))
    used = np.unique(oi)
    local = np.searchsorted(used, oi).astype(np.int32)
    pick = lambda p: (arrays[f"{p}_codes"][used], arrays[f"{p}_scales"][used].astype(np.float32))  # noqa: E731
    want = cpu.moe_decode(x.float().cpu().numpy(), local, r.weight.cpu().numpy(), pick("w1"), pick("w3"), pick("w2"),
                          e8p.e8p_packed_abs_grid())
    err = ops.max_rel_err(out.cpu().numpy(), want)
    assert err <= 2e-3, f"max rel err {err:.3e}"


def _residual(rng, n_hot):
    def res(N, Kd):
        c = rng.integers(0, 256, (n_hot, N, Kd // 8), dtype=np.uint8)
        s = (np.exp(rng.normal(0, 0.3, (n_hot, N, 1))) * 0.1).astype(np.float16)
        return c, s
    return {"gate": res(I, H), "up": res(I, H), "down": res(H, I)}


def _check(out, want, tol=2e-3):
    g = out.float().cpu().numpy()
    err = ops.max_rel_err(g, want)
    assert err <= tol, f"max rel err {err:.3e}"
    assert ops.elementwise_ok(g, want, rtol=tol), "elementwise bound violated"


@pytest.mark.parametrize("one_launch", [False, True])
def test_hot_tier_rows_follow_the_residents(dev, tmp_path, one_launch):
    """The nested tier over an 8-row pool: the cache's route hook rewrites the
    tier's slot rows as experts move (omlx_lattice.py:274-278). Hot experts 20
    and 27 start absent and are installed, one of them into the slot that hot
    expert 2 (never demanded, the coldest resident) held; expert 5 keeps its
    row throughout. Every call: each routed slot's tier row is its expert's row, and
    the fused nested layer matches the float64 oracle in expert space."""
    print(f"residency: hot tier rows follow the residents, one_launch={one_launch}", flush=True)
    arrays = _write_layer(tmp_path / "layer-00.npz")
    layer = loaders.LayerFile(tmp_path / "layer-00.npz")
    pools = _pools(dev)
    rng = np.random.default_rng(40)
    hot_row_of = {2: 0, 20: 1, 27: 2, 5: 3}
    residual = _residual(rng, len(hot_row_of))
    tier = keep_amd.HotTier(np.full(S, keep_amd.ops.NO_RESIDUAL, np.uint32),
                            {n: (torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev))
                             for n, (c, s) in residual.items()})
    order = [0, 1, 3, 4, 5, 6, 7, 2] + list(range(8, E))  # 2 in slot 7, the coldest: evicted first
    cache = ResidencyCache(loaders.ExpertInstaller(layer, pools, dev), E, order, tau=0.2, spare=1, lag=1,
                           hot_tier=tier, hot_row_of=hot_row_of)
    assert tier._hot32.cpu().tolist() == [-1, -1, -1, -1, 3, -1, -1, 0]
    hot_by_expert = np.full(E, keep_amd.ops.NO_RESIDUAL, np.uint32)
    for e, row in hot_row_of.items():
        hot_by_expert[e] = row
    proj = {p: (arrays[f"{p}_codes"], arrays[f"{p}_scales"]) for p in ("w1", "w3", "w2")}
    x = synth.rht_activations(1, H, seed=41, device=dev)
    served = set()
    for step in range(10):
        cache.begin()
        torch.cuda.synchronize()
        slot_expert = cache.table().slot_expert()
        rows, bits = tier._hot32.cpu().numpy(), tier.hot_of_slot.cpu().numpy().view(np.uint32)
        for s in cache.table().slots_in(ROUTED):
            want_row = hot_row_of.get(int(slot_expert[s]), -1)
            assert rows[s] == want_row and bits[s] == np.uint32(want_row & 0xFFFFFFFF), f"step {step} slot {s}"
        z_np = rng.standard_normal((1, E)).astype(np.float32)
        z_np[0, [20, 27]] += 6.0
        z_np[0, 2] -= 6.0
        z = torch.from_numpy(z_np).to(dev)
        out, r = keep_amd.moe_layer(x, z, pools["w1"], pools["w3"], pools["w2"], k=K, bias_served=cache.bias(),
                                    tau=cache.tau, slot_map=cache.slots(), hot_tier=tier, limit=7.0,
                                    one_launch=one_launch,
                                    workspace=keep_amd.nn.layer_workspace(dev, K, I) if one_launch else None)
        cache.observe(r)
        experts = slot_expert[r.idx.cpu().numpy()]
        assert (experts >= 0).all()
        served |= set(experts.ravel().tolist())
        want = ops.moe_layer(x.float().cpu().numpy(), experts, r.weight.cpu().numpy(), proj["w1"], proj["w3"],
                             proj["w2"], limit=7.0, h_round="bfloat16", hot_of_slot=hot_by_expert, residual=residual)
        _check(out, want)
    assert {20, 27} <= served and 2 not in cache.table().assignment()
    assert cache.mismatched() == 0


def test_prefill_in_pieces_over_the_slots(dev, tmp_path):
    """Prefill under the wait rule (omlx_lattice.py:427-449) over an 8-row
    pool: 24 tokens whose demand spans more experts than slots run in pieces;
    each piece fetches its demand (wait_min 0: every route), then RoutedVQMoE
    serves exactly that demand from the slots, against the C oracle on the
    piece's tokens. The next piece's copies queue behind the last run."""
    print("residency: prefill in pieces", flush=True)
    arrays = _write_layer(tmp_path / "layer-00.npz")
    layer = loaders.LayerFile(tmp_path / "layer-00.npz")
    pools = _pools(dev)
    cache = ResidencyCache(loaders.ExpertInstaller(layer, pools, dev), E, list(range(E)), tau=float("inf"), lag=1)

    def lin(p, Kd, N):
        return keep_amd.QuantizedVQSwitchLinear(input_dims=Kd, output_dims=N, num_experts=S, codes=pools[p][0],
                                                scales=pools[p][1], group_size=Kd, code_bits=16)
    glu = keep_amd.QuantizedVQSwitchGLU(gate_proj=lin("w1", H, I), up_proj=lin("w3", H, I),
                                        down_proj=lin("w2", I, H))
    moe = keep_amd.RoutedVQMoE(glu, top_k=K, bias_served=cache.bias(), slot_map=cache.slots())
    T = 24
    x = synth.rht_activations(T, H, seed=51, device=dev)
    z = synth.router_logits(T, E, seed=52, device=dev)
    demand = keep_amd.router_dual_topk(z, K)
    want, score = demand.want.cpu().numpy(), demand.want_score.cpu().numpy()
    host = {p: (arrays[f"{p}_codes"], arrays[f"{p}_scales"].astype(np.float32)) for p in ("w1", "w3", "w2")}
    ran = []

    def run(a, b):
        slot_expert = cache.table().slot_expert()
        out, r = moe(x[a:b], z[a:b])
        experts = slot_expert[r.idx.cpu().numpy()]
        np.testing.assert_array_equal(np.sort(experts, 1), np.sort(want[a:b], 1))
        used = np.unique(experts)
        local = np.searchsorted(used, experts).astype(np.int32)
        pick = lambda p: (host[p][0][used], host[p][1][used])  # noqa: E731
        ref = cpu.moe_decode(x[a:b].float().cpu().numpy(), local, r.weight.cpu().numpy(), pick("w1"), pick("w3"),
                             pick("w2"), e8p.e8p_packed_abs_grid())
        err = ops.max_rel_err(out.float().cpu().numpy(), ref)
        assert err <= 2e-3, f"piece {a}:{b}: max rel err {err:.3e}"
        ran.append((a, b))
    n = cache.run_pieces(want, score, 0.0, run)
    assert n >= 3 and ran[0][0] == 0 and ran[-1][1] == T and all(p[1] == q[0] for p, q in zip(ran, ran[1:]))
    assert cache.stats["waits"] >= n - 1 and cache.mismatched() == 0


def test_slot_bytes_check_and_stats_log(dev, tmp_path):
    """The stats log's byte check (omlx_routed.py:138-145,249-260): a routed
    slot whose device bytes differ from its expert's stored bytes counts."""
    _write_layer(tmp_path / "layer-00.npz")
    layer = loaders.LayerFile(tmp_path / "layer-00.npz")
    pools = _pools(dev)
    cache = ResidencyCache(loaders.ExpertInstaller(layer, pools, dev), E, list(range(E)), tau=0.2, spare=1, lag=1)
    assert cache.mismatched() == 0
    pools["w2"][1][3, 7, 0] += 1.0  # one scale of slot 3
    assert cache.differing(0, 3) == 1 and cache.differing(0, 2) == 0
    row = cache.write_log(tmp_path / "stats.jsonl", verify=True)
    assert row["mismatched"] == 1 and row["step"] == 0


def test_one_policy_over_two_layers(dev, tmp_path):
    """One clock over two layers' pools: begin() once per forward, each
    layer's demand observed after its call; each layer installs its own
    strongly demanded expert into its own pool, and the routed layers serve
    from their own slot maps."""
    print("residency: two layers", flush=True)
    files, pools = [], []
    for li in range(2):
        _write_layer(tmp_path / f"layer-{li:02d}.npz")
        files.append(loaders.LayerFile(tmp_path / f"layer-{li:02d}.npz"))
        pools.append(_pools(dev))
    cache = ResidencyCache.for_layers(
        [(loaders.ExpertInstaller(files[li], pools[li], dev), E, list(range(E)) if li == 0 else list(range(E))[::-1])
         for li in range(2)], tau=0.2, spare=1, lag=1)
    hot = {0: 25, 1: 3}  # absent at first in each layer (layer 1 starts with 31..24)
    rng = np.random.default_rng(60)
    x = synth.rht_activations(1, H, seed=61, device=dev)
    for _ in range(6):
        cache.begin()
        for li in range(2):
            z_np = rng.standard_normal((1, E)).astype(np.float32)
            z_np[0, hot[li]] += 6.0
            _, r = keep_amd.moe_layer(x, torch.from_numpy(z_np).to(dev), pools[li]["w1"], pools[li]["w3"],
                                      pools[li]["w2"], k=K, bias_served=cache.bias(li), tau=cache.tau,
                                      slot_map=cache.slots(li))
            cache.observe(r, li)
    torch.cuda.synchronize()
    for li in range(2):
        assert hot[li] in cache.table(li).assignment()
        assert cache.bias(li)[hot[li]].item() == 0.0
        assert cache.slots(li)[hot[li]].item() == cache.table(li).assignment()[hot[li]]
    assert cache.mismatched() == 0
