"""GPU parity of the prefill grouped GEMM (keep_vq_grouped_gemm_q8, fp16
matrix cores) and its fused gate/up + SwiGLU form (keep_vq_grouped_swiglu_q8)
against the float64 oracle: partial column blocks, tiles of one and two
32-route m-tiles, per-row and grouped scales, fp16 / bf16 / fp32
activations, work items of 256 and of 512 columns, the scatter back to route
order, and NaN rows / out-of-range experts (the sorted-route prefill of
src/ramp/ops/vq_switch.py:620-913 and src/ramp/models/glm4_moe_adapter.py:274-353)."""

import numpy as np
import pytest
import torch

import keep_amd
from keep_amd import ops as kops
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


def _plan(rhs, E, k, dev):
    flat = _t(rhs.reshape(-1).astype(np.int32), dev)
    order, inverse, counts, _, te, to, tc, _ = keep_amd.route_plan(flat, E, 64)
    lhs = (torch.arange(flat.numel(), device=dev, dtype=torch.int32) // k)[order.long()].contiguous()
    return flat, order, inverse, counts, (te, to, tc), lhs


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("G", [1, 4])
def test_grouped_gemm_q8_vs_oracle(dev, xdt, G):
    """N = 320: a full and a partial 256-column block; Zipf routing gives
    experts with > 64, 33..64 and <= 32 routes."""
    E, N, K, T, k = 12, 320, 512, 100, 4
    codes, scales = synth.projection_np(E, N, K, group_size=K // G, seed=G)
    rhs = synth.zipf_routes(T, E, k, seed=3)
    x = synth.rht_activations(T, K, seed=4, device=dev, dtype=xdt)
    flat, order, inverse, counts, tiles, lhs = _plan(rhs, E, k, dev)
    c = counts.cpu().numpy()
    assert c.max() > 64 and ((c > 32) & (c <= 64)).any() and ((c > 0) & (c <= 32)).any()
    cb = kops._default_codebook(16, dev)
    want = ops.gather_token(x.float().cpu().numpy(), codes, scales, rhs)
    y = kops.grouped_gemm(x, _t(codes, dev), _t(scales, dev), cb, tiles, lhs=lhs, routes=flat.numel(),
                          input_dims=K, output_dims=N, group_size=K // G, out_dtype=torch.float32)
    _check(y[inverse.long()].reshape(T, k, N), want)
    # the same rows scattered straight to route order
    y2 = kops.grouped_gemm(x, _t(codes, dev), _t(scales, dev), cb, tiles, lhs=lhs, routes=flat.numel(),
                           input_dims=K, output_dims=N, group_size=K // G, out_dtype=torch.float32, out_index=order)
    assert torch.equal(y2, y[inverse.long()])


@pytest.mark.parametrize("limit", [0.0, 7.0])
def test_grouped_swiglu_q8_vs_oracle(dev, limit):
    """I = 320: two full 128-row blocks and a partial one."""
    E, H, I, T, k = 10, 512, 320, 60, 3
    gate = synth.projection_np(E, I, H, seed=31)
    up = synth.projection_np(E, I, H, seed=32)
    rhs = synth.zipf_routes(T, E, k, seed=33)
    x = synth.rht_activations(T, H, seed=34, device=dev)
    flat, order, inverse, _, tiles, lhs = _plan(rhs, E, k, dev)
    cb = kops._default_codebook(16, dev)
    h = kops.grouped_swiglu(x, _t(gate[0], dev), _t(gate[1], dev), _t(up[0], dev), _t(up[1], dev), cb, tiles,
                            lhs=lhs, routes=flat.numel(), input_dims=H, hidden_dims=I, group_size=H, limit=limit)
    xf = x.float().cpu().numpy()
    g = ops.gather_token(xf, gate[0], gate[1], rhs)
    u = ops.gather_token(xf, up[0], up[1], rhs)
    want = ops.round_bf16(ops.swiglu(g, u, limit))
    # bf16-stored h on both sides: two nearly equal values can round one bf16
    # ulp apart, 2**-7 of the smaller where they straddle a power of two
    _check(h[inverse.long()].reshape(T, k, I), want, TOL + 2.0 ** -7)


def test_grouped_gemm_q8_nan_row_and_bad_expert(dev):
    E, N, K, T, k = 4, 256, 256, 40, 2
    codes, scales = synth.projection_np(E, N, K, seed=41)
    rng = np.random.default_rng(42)
    rhs = rng.integers(0, E, size=(T, k)).astype(np.int32)
    rhs[5, 1] = 7  # out of range: its route's row is NaN
    x = synth.rht_activations(T, K, seed=43, device=dev)
    x[9, 17] = float("nan")  # token 9's routes are NaN
    flat = _t(rhs.reshape(-1), dev)
    order, inverse, _, _, te, to, tc, _ = keep_amd.route_plan(flat, E, 64)  # expert 7: a tile of expert -1
    lhs = (torch.arange(flat.numel(), device=dev, dtype=torch.int32) // k)[order.long()].contiguous()
    cb = kops._default_codebook(16, dev)
    y = kops.grouped_gemm(x, _t(codes, dev), _t(scales, dev), cb, (te, to, tc), lhs=lhs, routes=flat.numel(),
                          input_dims=K, output_dims=N, group_size=K, out_dtype=torch.float32,
                          out_index=order).reshape(T, k, N).cpu()
    bad = np.zeros((T, k), dtype=bool)
    bad[5, 1] = True
    bad[9, :] = True
    assert torch.isnan(y[torch.from_numpy(bad)]).all()
    good = ~bad
    assert not torch.isnan(y[torch.from_numpy(good)]).any()
    rr = np.where(rhs < E, rhs, 0)
    want = ops.gather_token(np.nan_to_num(x.float().cpu().numpy()), codes, scales, rr)
    _check(y[torch.from_numpy(good)], want[good])


@pytest.mark.parametrize("G", [1, 2])
def test_grouped_residual_add_vs_oracle(dev, G):
    """The 8-bit E8 residual form: tiles of routes grouped by residual row
    (route_plan over the routes' rows, -1 = none, sorted past every tile) add
    R[row] . x into an fp32 output at out_index; routes off the tier keep
    their value."""
    from oracle import e8p

    Hh, N, K, T, k = 5, 320, 512, 60, 3
    rng = np.random.default_rng(101)
    rc = rng.integers(0, 256, (Hh, N, K // 8), dtype=np.uint8)
    rs = (np.exp(rng.normal(0, 0.3, (Hh, N, G))) * 0.1).astype(np.float16)
    dense = e8p.decode_e8_1bit(rc).astype(np.float64).reshape(Hh, N, K) * np.repeat(rs.astype(np.float64), K // G, -1)
    rows = rng.integers(-1, Hh, size=T * k).astype(np.int32)
    x = synth.rht_activations(T, K, seed=102, device=dev)
    flat = _t(rows, dev)
    order, _, _, _, te, to, tc, _ = keep_amd.route_plan(flat, Hh, 64)
    lhs = (torch.arange(T * k, device=dev, dtype=torch.int32) // k)[order.long()].contiguous()
    base = torch.randn(T * k, N, device=dev)
    out = base.clone()
    kops.grouped_residual_add(out, x, _t(rc, dev), _t(rs, dev), (te, to, tc), lhs=lhs, out_index=order,
                              routes=T * k, input_dims=K, output_dims=N, group_size=K // G)
    xf = x.float().cpu().numpy().astype(np.float64)
    want = np.stack([dense[r] @ xf[i // k] if r >= 0 else np.zeros(N) for i, r in enumerate(rows)])
    got = (out - base).cpu().numpy()
    assert (got[rows < 0] == 0).all()
    assert ops.max_rel_err(got, want) <= TOL


def test_out_of_range_route_is_nan_through_gather_and_glu(dev):
    """R >= 128 takes the sorted-route GEMM: a route whose expert is out of
    range sorts past every valid tile and its row comes back NaN (not
    unwritten memory), through gather_vqmm and through the shared-plan
    prefill of QuantizedVQSwitchGLU; every other row matches the oracle."""
    from keep_amd.nn import QuantizedVQSwitchGLU, QuantizedVQSwitchLinear

    E, H, I, T, k = 6, 256, 256, 48, 4
    gate, up, down = (synth.projection_np(E, I, H, seed=61), synth.projection_np(E, I, H, seed=62),
                      synth.projection_np(E, H, I, seed=63))
    rng = np.random.default_rng(64)
    rhs = rng.integers(0, E, size=(T, k)).astype(np.int32)
    rhs[3, 2], rhs[17, 0], rhs[40, 3] = E, -1, E + 9
    bad = (rhs < 0) | (rhs >= E)
    x = synth.rht_activations(T, H, seed=65, device=dev)
    for trial in range(2):  # the output buffer of the second call is recycled memory
        y = kops.gather_vqmm(x, _t(gate[0], dev), _t(gate[1], dev), None, _t(rhs, dev), input_dims=H,
                             output_dims=I, group_size=H, code_bits=16)
        assert y.shape == (T, k, I)
        yc = y.float().cpu()
        assert torch.isnan(yc[torch.from_numpy(bad)]).all()
        assert not torch.isnan(yc[torch.from_numpy(~bad)]).any()
    want = ops.gather_token(x.float().cpu().numpy(), gate[0], gate[1], np.where(bad, 0, rhs))
    _check(yc[torch.from_numpy(~bad)], want[~bad])

    def lin(p, K, N):
        return QuantizedVQSwitchLinear(input_dims=K, output_dims=N, num_experts=E, codes=_t(p[0], dev),
                                       scales=_t(p[1], dev), group_size=K, code_bits=16)

    glu = QuantizedVQSwitchGLU(gate_proj=lin(gate, H, I), up_proj=lin(up, H, I), down_proj=lin(down, I, H))
    out = glu(x, _t(rhs, dev)).float().cpu()
    assert out.shape == (T, k, H)
    assert torch.isnan(out[torch.from_numpy(bad)]).all()
    assert not torch.isnan(out[torch.from_numpy(~bad)]).any()


def test_grouped_gemm_q8_blocks_run_many_items(dev):
    """More work items than blocks: at N = 2048 (eight 256-column blocks)
    and ~100 tiles every persistent block runs two or more non-empty items
    back to back, so a block's next item must not overwrite the row scales
    and output rows that its lagging waves still read in the previous
    item's epilogue. Checked against the C oracle on every route."""
    from oracle import cpu

    E, N, K, T, k = 40, 2048, 512, 1200, 4
    codes, scales = synth.projection_np(E, N, K, seed=71)
    rhs = synth.zipf_routes(T, E, k, s=1.1, seed=72)
    x = synth.rht_activations(T, K, seed=73, device=dev)
    flat, order, inverse, counts, tiles, lhs = _plan(rhs, E, k, dev)
    n_tiles = int((tiles[2] > 0).sum().item())
    assert n_tiles * (N // 256) > 2 * 256, "fewer work items than two per block"
    cb = kops._default_codebook(16, dev)
    y = kops.grouped_gemm(x, _t(codes, dev), _t(scales, dev), cb, tiles, lhs=lhs, routes=flat.numel(),
                          input_dims=K, output_dims=N, group_size=K, out_dtype=torch.float32, out_index=order)
    want = cpu.routed_matvec(x.float().cpu().numpy(), codes, scales.astype(np.float32),
                             kops.e8p_packed_abs_grid(), rhs.reshape(-1), x_div=k, group_size=K)
    _check(y, want.astype(np.float64))


@pytest.mark.parametrize("G", [1, 2])
@pytest.mark.parametrize("form", ["plain", "swiglu"])
def test_grouped_gemm_wide_items(dev, form, G):
    """Enough route tiles for work items of 512 columns (two n-tiles per
    wave): 160 experts with ~32 routes each (tiles of one and two m-tiles),
    N = 4096 (plain) or I = 2048 (gate/up + SwiGLU), per-row and grouped
    scales, against the C oracle's fp32 row dots."""
    E, K, T, k = 160, 256, 2560, 2
    rng = np.random.default_rng(50 + G)
    rhs = rng.integers(0, E, (T, k)).astype(np.int32)
    x = synth.rht_activations(T, K, seed=51, device=dev)
    flat, order, inverse, counts, tiles, lhs = _plan(rhs, E, k, dev)
    c = counts.cpu().numpy()
    assert tiles[0].numel() >= 128 and (c > 32).any() and ((c > 0) & (c <= 32)).any()
    cb = kops._default_codebook(16, dev)
    tab = e8p.e8p_packed_abs_grid()
    xf = x.float().cpu().numpy()
    R = flat.numel()

    def oracle(codes, scales):
        return cpu.routed_matvec(xf, codes, scales.astype(np.float32), tab, rhs.reshape(-1), x_div=k,
                                 group_size=K // G).astype(np.float64)
    if form == "plain":
        N = 4096
        codes, scales = synth.projection_np(E, N, K, group_size=K // G, seed=52)
        y = kops.grouped_gemm(x, _t(codes, dev), _t(scales, dev), cb, tiles, lhs=lhs, routes=R, input_dims=K,
                              output_dims=N, group_size=K // G, out_dtype=torch.float32)
        _check(y[inverse.long()], oracle(codes, scales))
    else:
        I = 2048
        gate = synth.projection_np(E, I, K, group_size=K // G, seed=53)
        up = synth.projection_np(E, I, K, group_size=K // G, seed=54)
        h = kops.grouped_swiglu(x, _t(gate[0], dev), _t(gate[1], dev), _t(up[0], dev), _t(up[1], dev), cb, tiles,
                                lhs=lhs, routes=R, input_dims=K, hidden_dims=I, group_size=K // G, limit=7.0)
        with np.errstate(over="ignore"):
            want = ops.round_bf16(ops.swiglu(oracle(*gate), oracle(*up), limit=7.0))
        got = h[inverse.long()].float().cpu().numpy()
        assert ops.elementwise_ok(got, want, rtol=TOL + 2.0 ** -7), "h beyond one bf16 ulp of the oracle's"
