"""keep_moe_layer_noalloc through the C ABI: the routed decode layer with h in
the library's static device scratch instead of a caller's h_work. Its outputs
(router outputs and layer output) must equal keep_moe_layer's bit for bit on
the same inputs, over consecutive calls that shrink the shape (the scratch
keeps the previous call's contents), and a shape beyond the scratch is
refused before anything launches."""

import pytest
import torch

from keep_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
SCRATCH_H = 12288  # k * I bf16 values the static scratch holds


def _layer_args(dev, E, I, k, seed, xdt=torch.float16):
    H = 4096
    gate = synth.projection(E, I, H, seed=seed, device=dev)
    up = synth.projection(E, I, H, seed=seed + 1, device=dev)
    down = synth.projection(E, H, I, seed=seed + 2, device=dev)
    x = synth.rht_activations(1, H, seed=seed + 3, device=dev, dtype=xdt)
    z = synth.router_logits(1, E, seed=seed + 4, device=dev)
    return dict(E=E, I=I, k=k, H=H, gate=gate, up=up, down=down, x=x, z=z,
                prep=ops.prepared_table(ops._codebook_tensor(None, 16, dev)))


def _outputs(dev, k, H):
    return dict(idx=torch.full((1, k), -7, dtype=torch.int32, device=dev),
                w=torch.full((1, k), -7.0, dtype=torch.float32, device=dev),
                want=torch.full((1, k), -7, dtype=torch.int32, device=dev),
                want_score=torch.full((1, k), -7.0, dtype=torch.float32, device=dev),
                admit=torch.full((1, k), 7, dtype=torch.uint8, device=dev),
                out=torch.full((1, H), float("nan"), dtype=torch.float32, device=dev))


def _call(name, a, o, h_work=None):
    lib = _lib.load()
    g, u, d = a["gate"], a["up"], a["down"]
    head = [a["z"].data_ptr(), None, None, _lib.SCORE_FUNCS["softmax"], 1, 1.0, float("inf"), None, 0, a["E"], a["k"],
            a["x"].data_ptr(), ops._DT[a["x"].dtype], a["H"], a["I"], g.codes.data_ptr(), g.scales.data_ptr(),
            u.codes.data_ptr(), u.scales.data_ptr(), d.codes.data_ptr(), d.scales.data_ptr(),
            ops._DT[g.scales.dtype], a["H"], a["I"], a["prep"].data_ptr(), 0.0, o["idx"].data_ptr(),
            o["w"].data_ptr(), o["want"].data_ptr(), o["want_score"].data_ptr(), o["admit"].data_ptr()]
    tail = [o["out"].data_ptr(), ops._DT[torch.float32], torch.cuda.current_stream().cuda_stream]
    mid = [] if h_work is None else [h_work.data_ptr()]
    return getattr(lib, name)(*head, *mid, *tail)


def _same(a, b):
    for key in ("idx", "w", "want", "want_score", "admit", "out"):
        assert torch.equal(a[key], b[key]), f"{key} differs from keep_moe_layer's"


@pytest.mark.parametrize("shapes", [[(384, 2048, 6, 1), (64, 1024, 4, 11), (288, 1536, 8, 21)]])
def test_noalloc_layer_matches_keep_moe_layer(dev, shapes):
    for E, I, k, seed in shapes:
        print(f"noalloc layer: E={E} I={I} k={k} seed={seed}", flush=True)
        assert k * I <= SCRATCH_H
        a = _layer_args(dev, E, I, k, seed)
        ref, got = _outputs(dev, k, 4096), _outputs(dev, k, 4096)
        h_work = torch.empty(k * I, dtype=torch.bfloat16, device=dev)
        assert _call("keep_moe_layer", a, ref, h_work) == 0, _lib.load().keep_last_error()
        assert _call("keep_moe_layer_noalloc", a, got) == 0, _lib.load().keep_last_error()
        torch.cuda.synchronize()
        assert not torch.isnan(got["out"]).any()
        _same(ref, got)


def test_noalloc_layer_refuses_shapes_beyond_its_scratch(dev):
    a = _layer_args(dev, 64, 2048, 8, 31)  # k * I = 16384 > 12288
    o = _outputs(dev, 8, 4096)
    rc = _call("keep_moe_layer_noalloc", a, o)
    assert rc == _lib.KEEP_EINVAL
    assert b"static scratch" in _lib.load().keep_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(o["out"]).all(), "nothing may launch for a refused shape"
