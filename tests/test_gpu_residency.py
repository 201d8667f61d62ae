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
from keep_amd.residency import ResidencyCache
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
        slot_expert = cache.slot_expert.copy()
        resident = cache.resident_mask()
        for s, e in enumerate(slot_expert):  # every routed row holds its expert's file bytes
            if e >= 0:
                np.testing.assert_array_equal(pools["w1"][0][s].cpu().numpy().view(np.uint16), arrays["w1_codes"][e])
                np.testing.assert_array_equal(pools["w2"][0][s].cpu().numpy().view(np.uint16), arrays["w2_codes"][e])
        z_np = rng.standard_normal((1, E)).astype(np.float32)
        z_np[0, hot] += 6.0
        z = torch.from_numpy(z_np).to(dev)
        out, r = keep_amd.moe_layer(x, z, pools["w1"], pools["w3"], pools["w2"], k=K,
                                    bias_served=cache.bias_served, tau=cache.tau, slot_map=cache.slot_map,
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
    assert all(h in cache.slot_of for h in hot), "strongly demanded experts are resident by now"
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
        cache.pending.setdefault(cache.step, []).append((want, score))
    assert 30 in cache.reading and 30 not in cache.slot_of
    assert cache.bias_served[30].item() <= ops.MASKED_BIAS
    cache.hold = False
    torch.cuda.synchronize()
    cache.begin()
    torch.cuda.synchronize()
    slot = cache.slot_of[30]
    assert cache.bias_served[30].item() == 0.0 and cache.slot_map[30].item() == slot
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
    moe = keep_amd.RoutedVQMoE(glu, top_k=K, bias_served=cache.bias_served, slot_map=cache.slot_map)
    x = synth.rht_activations(T, H, seed=T, device=dev)
    z = synth.router_logits(T, E, seed=T + 1, device=dev)
    out, r = moe(x, z)
    bias = np.where(cache.resident_mask(), 0.0, ops.MASKED_BIAS)
    oi, ow, *_ = ops.router_dual_topk(z.cpu().numpy(), bias, np.zeros(E), K)
    np.testing.assert_array_equal(r.idx.cpu().numpy(), np.vectorize(cache.slot_of.get)(oi))
    used = np.unique(oi)
    local = np.searchsorted(used, oi).astype(np.int32)
    pick = lambda p: (arrays[f"{p}_codes"][used], arrays[f"{p}_scales"][used].astype(np.float32))  # noqa: E731
    want = cpu.moe_decode(x.float().cpu().numpy(), local, r.weight.cpu().numpy(), pick("w1"), pick("w3"), pick("w2"),
                          e8p.e8p_packed_abs_grid())
    err = ops.max_rel_err(out.cpu().numpy(), want)
    assert err <= 2e-3, f"max rel err {err:.3e}"
