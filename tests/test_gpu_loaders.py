"""Device loads from the on-disk formats and expert installs into slot rows.

Files are written as the reference writes them (``np.savez`` of stacked
``{w1,w3,w2}_{codes,scales}`` plus ``code_bits``; safetensors with a codebook
hash in ``quantization_config``). The device bytes must equal the file's, and
a routed MoE built from the loaded module must equal, bit for bit, the one
built from the same arrays in memory."""

import json

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

E, H, I, K_TOP, T = 16, 512, 256, 4, 2


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda", 0)


def _write_layer(path):
    from keep_amd import synth

    arrays = {}
    for proj, (n, k), seed in (("w1", (I, H), 1), ("w3", (I, H), 2), ("w2", (H, I), 3)):
        codes, scales = synth.projection_np(E, n, k, seed=seed)
        arrays[f"{proj}_codes"], arrays[f"{proj}_scales"] = codes, scales
    np.savez(path, code_bits=np.asarray(16), **arrays)
    return arrays


def _as_u16(t):
    return t.cpu().numpy().view(np.uint16)


def test_npz_layer_loads_bit_exact(dev, tmp_path):
    import keep_amd
    from keep_amd import loaders, synth

    print("loaders: npz layer", flush=True)
    arrays = _write_layer(tmp_path / "layer-00.npz")
    glu = loaders.load_switch_glu_npz(tmp_path / "layer-00.npz", device=dev)
    for role, proj in loaders.PROJECTIONS:
        lin = getattr(glu, f"{role}_proj")
        np.testing.assert_array_equal(_as_u16(lin.codes), arrays[f"{proj}_codes"])
        np.testing.assert_array_equal(lin.scales.cpu().numpy(), arrays[f"{proj}_scales"])

    def mk(c, s, k):
        return keep_amd.QuantizedVQSwitchLinear(input_dims=k, output_dims=c.shape[1], num_experts=E,
                                                codes=torch.from_numpy(c.view(np.int16)).to(dev),
                                                scales=torch.from_numpy(s).to(dev), group_size=k, code_bits=16)

    ref = keep_amd.QuantizedVQSwitchGLU(gate_proj=mk(arrays["w1_codes"], arrays["w1_scales"], H),
                                        up_proj=mk(arrays["w3_codes"], arrays["w3_scales"], H),
                                        down_proj=mk(arrays["w2_codes"], arrays["w2_scales"], I))
    x = synth.rht_activations(T, H, seed=9, device=dev)
    logits = synth.router_logits(T, E, seed=10, device=dev)
    out_a, r_a = keep_amd.RoutedVQMoE(glu, top_k=K_TOP)(x, logits)
    out_b, r_b = keep_amd.RoutedVQMoE(ref, top_k=K_TOP)(x, logits)
    torch.cuda.synchronize()
    assert torch.equal(r_a.idx, r_b.idx)
    assert torch.equal(out_a, out_b)

    sub = loaders.load_switch_glu_npz(tmp_path / "layer-00.npz", device=dev, experts=[5, 1, 3])
    np.testing.assert_array_equal(_as_u16(sub.down_proj.codes), arrays["w2_codes"][[5, 1, 3]])


def test_safetensors_switch_linear(dev, tmp_path):
    from safetensors.numpy import save_file

    from keep_amd import loaders, synth

    print("loaders: safetensors", flush=True)
    codes, scales = synth.projection_np(E, I, H, group_size=128, seed=4)
    meta = {"quantization_config": json.dumps({"codebook": {"sha256": loaders.codebook_sha256(16)}})}
    p = tmp_path / "m.safetensors"
    save_file({"layers.0.mlp.experts.gate_proj.codes": codes, "layers.0.mlp.experts.gate_proj.scales": scales},
              str(p), metadata=meta)
    lin = loaders.load_switch_linear_safetensors(p, "layers.0.mlp.experts.gate_proj", device=dev)
    assert (lin.input_dims, lin.output_dims, lin.num_experts, lin.group_size, lin.code_bits) == (H, I, E, 128, 16)
    np.testing.assert_array_equal(_as_u16(lin.codes), codes)
    np.testing.assert_array_equal(lin.scales.cpu().numpy(), scales)


def test_expert_installer_fills_slots(dev, tmp_path):
    from keep_amd import loaders

    print("loaders: installer", flush=True)
    arrays = _write_layer(tmp_path / "layer-01.npz")
    lf = loaders.LayerFile(tmp_path / "layer-01.npz")
    S = 4
    pools = {proj: (torch.zeros((S, *arrays[f"{proj}_codes"].shape[1:]), dtype=torch.int16, device=dev),
                    torch.zeros((S, *arrays[f"{proj}_scales"].shape[1:]), dtype=torch.float16, device=dev))
             for proj in ("w1", "w3", "w2")}
    inst = loaders.ExpertInstaller(lf, pools, dev)
    events = [inst.submit(11, 2), inst.submit(6, 0)]
    for ev in events:
        ev.synchronize()
        assert inst.ready(ev)
    for proj, (codes, scales) in pools.items():
        c = _as_u16(codes)
        np.testing.assert_array_equal(c[2], arrays[f"{proj}_codes"][11])
        np.testing.assert_array_equal(c[0], arrays[f"{proj}_codes"][6])
        assert not c[1].any() and not c[3].any()
        np.testing.assert_array_equal(scales.cpu().numpy()[2], arrays[f"{proj}_scales"][11])
    with pytest.raises(IndexError):
        inst.submit(1, S)
    # a pool whose dtype would reinterpret the file's bits is refused
    bad = dict(pools)
    bad["w2"] = (pools["w2"][0], pools["w2"][1].to(torch.bfloat16))
    with pytest.raises(ValueError, match="file's"):
        loaders.ExpertInstaller(lf, bad, dev)
