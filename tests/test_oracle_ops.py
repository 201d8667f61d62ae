"""Pins the dense oracle operators against brute force, closed forms and the
router semantics of the reference (tests/test_runpod_v41_routed_precision.py:158-179)."""

import numpy as np
import pytest
import scipy.linalg

from oracle import cpu, e8p, ops, rht


def _proj(E, N, K, G, seed):
    rng = np.random.default_rng(seed)
    return (rng.integers(0, 1 << 16, size=(E, N, K // 8), dtype=np.uint16),
            np.exp(rng.normal(0, 0.3, size=(E, N, G))).astype(np.float16))


def _brute_row(codes_row, scales_row, x):
    """Scalar loop over codewords and dims with the bitwise decoder."""
    C = codes_row.shape[0]
    G = scales_row.shape[0]
    total = 0.0
    for c in range(C):
        vals = e8p.decode_e8p_scalar(int(codes_row[c]))
        s = float(scales_row[c // (C // G)])
        for d in range(8):
            total += vals[d] * s * float(x[8 * c + d])
    return total


def test_qmv_matches_scalar_brute_force():
    codes, scales = _proj(1, 5, 64, 2, 0)
    x = np.random.default_rng(1).standard_normal(64)
    y = ops.qmv(x, codes[0], scales[0])
    want = [_brute_row(codes[0, n], scales[0, n], x) for n in range(5)]
    np.testing.assert_allclose(y, want, rtol=1e-12, atol=1e-12)


def test_gather_layouts_and_linearity():
    codes, scales = _proj(4, 6, 32, 1, 2)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 32))
    rhs = np.array([[0, 3], [2, 2], [1, 0]])
    tok = ops.gather_token(x, codes, scales, rhs)
    per = ops.gather_routes(x, codes, scales, rhs.reshape(-1), np.repeat(np.arange(3), 2))
    np.testing.assert_array_equal(tok.reshape(6, 6), per)
    for t in range(3):
        for j in range(2):
            np.testing.assert_allclose(tok[t, j], ops.qmv(x[t], codes[rhs[t, j]], scales[rhs[t, j]]), rtol=1e-13)
    # linearity in x
    a, b = rng.standard_normal(32), rng.standard_normal(32)
    np.testing.assert_allclose(ops.qmv(2 * a - b, codes[1], scales[1]),
                               2 * ops.qmv(a, codes[1], scales[1]) - ops.qmv(b, codes[1], scales[1]), atol=1e-10)


def test_nested_is_base_plus_residual():
    codes, scales = _proj(3, 4, 32, 1, 4)
    rng = np.random.default_rng(5)
    rc = rng.integers(0, 256, size=(2, 4, 4), dtype=np.uint8)
    rs = np.exp(rng.normal(0, 0.3, size=(2, 4, 1))).astype(np.float16)
    hot = np.array([ops.NO_RESIDUAL, 1, 0], dtype=np.uint32)
    x = rng.standard_normal((3, 32))
    rhs, lhs = np.array([0, 1, 2]), np.array([0, 1, 2])
    y = ops.nested_routes(x, (codes, scales), (rc, rs), hot, rhs, lhs)
    base = ops.gather_routes(x, codes, scales, rhs, lhs)
    np.testing.assert_array_equal(y[0], base[0])
    res1 = ops.dense(rc[1], rs[1], code_bits=8) @ x[1]
    np.testing.assert_allclose(y[1], base[1] + res1, rtol=1e-13)


def test_score_functions_closed_form():
    z = np.array([[-3.0, 0.0, 2.5, 40.0]])
    np.testing.assert_allclose(ops.score(z, "softmax"), np.exp(z - 40) / np.exp(z - 40).sum(), rtol=1e-14)
    np.testing.assert_allclose(ops.score(z, "sigmoid"), 1 / (1 + np.exp(-z)), rtol=1e-14)
    np.testing.assert_allclose(ops.score(z, "sqrtsoftplus"), np.sqrt(np.log1p(np.exp(z))), rtol=1e-12)


def test_topk_tie_rule_and_nan():
    keys = np.array([[1.0, 3.0, 3.0, np.nan, 2.0]])
    assert ops.topk_rule(keys, 3).tolist() == [[1, 2, 4]]
    assert ops.topk_rule(np.array([[-np.inf, -np.inf, 0.0]]), 3).tolist() == [[2, 0, 1]]


def test_router_identity_when_nothing_masked():
    rng = np.random.default_rng(0)
    z = rng.standard_normal((5, 16))
    idx, w, want, ws, admit = ops.router_dual_topk(z, np.zeros(16), np.zeros(16), 3, func="sqrtsoftplus",
                                                    route_scale=1.5)
    s = ops.score(z, "sqrtsoftplus")
    np.testing.assert_array_equal(idx, np.argsort(-s, axis=1, kind="stable")[:, :3])
    np.testing.assert_array_equal(idx, want)
    np.testing.assert_allclose(w.sum(-1), 1.5)
    assert not admit.any()


def test_router_masked_expert_rerouted_and_renormalised():
    rng = np.random.default_rng(1)
    z = rng.standard_normal((4, 8))
    idx0, *_ = ops.router_dual_topk(z, np.zeros(8), np.zeros(8), 3)
    bias = np.zeros(8)
    bias[idx0[0, 0]] = ops.MASKED_BIAS
    idx, w, want, ws, admit = ops.router_dual_topk(z, bias, np.zeros(8), 3, route_scale=1.5, tau=0.0)
    assert not (idx == idx0[0, 0]).any()
    np.testing.assert_allclose(w.sum(-1), 1.5)
    np.testing.assert_array_equal(want, idx0)  # demand ignores residency
    assert admit[0, 0] and (admit == (want == idx0[0, 0])).all()


def test_router_fewer_allowed_than_k_gives_zero_weight():
    rng = np.random.default_rng(2)
    z = rng.standard_normal((4, 8))
    bias = np.full(8, -np.inf)
    bias[:2] = 0
    idx, w, *_ = ops.router_dual_topk(z, bias, np.zeros(8), 3)
    assert ((w > 0).sum(-1) == 2).all() and (idx[w > 0] < 2).all()
    np.testing.assert_allclose(w.sum(-1), 1.0)


def test_swiglu_closed_form():
    g = np.array([-20.0, -1.0, 0.0, 3.0, 50.0])
    u = np.array([1.0, 2.0, 3.0, -40.0, 0.5])
    np.testing.assert_allclose(ops.swiglu(g, u), g * u / (1 + np.exp(-g)))
    lim = ops.swiglu(g, u, 10.0)
    gg, uu = np.minimum(g, 10), np.clip(u, -10, 10)
    np.testing.assert_allclose(lim, gg * uu / (1 + np.exp(-gg)))


def test_moe_layer_brute_force_tiny():
    E, H, I = 3, 16, 8
    gate, up, down = _proj(E, I, H, 1, 6), _proj(E, I, H, 1, 7), _proj(E, H, I, 1, 8)
    x = np.random.default_rng(9).standard_normal((1, H))
    idx = np.array([[2, 0]])
    w = np.array([[0.7, 0.3]])
    got = ops.moe_layer(x, idx, w, gate, up, down, limit=0.0)
    want = np.zeros(H)
    for j, e in enumerate(idx[0]):
        g = np.array([_brute_row(gate[0][e, n], gate[1][e, n], x[0]) for n in range(I)])
        u = np.array([_brute_row(up[0][e, n], up[1][e, n], x[0]) for n in range(I)])
        h = g / (1 + np.exp(-g)) * u
        want += w[0, j] * np.array([_brute_row(down[0][e, n], down[1][e, n], h) for n in range(H)])
    np.testing.assert_allclose(got[0], want, rtol=1e-10, atol=1e-12)


def test_route_plan_invariants():
    rng = np.random.default_rng(3)
    E, R, tile = 7, 50, 4
    rhs = rng.integers(0, E, size=R)
    order, inv, counts, offsets, te, to, tc = ops.route_plan(rhs, E, tile)
    assert sorted(order.tolist()) == list(range(R))
    assert np.all(np.diff(rhs[order]) >= 0)
    for e in range(E):  # stable: original order inside each expert
        pos = order[offsets[e]:offsets[e] + counts[e]]
        assert np.all(np.diff(pos) > 0)
    np.testing.assert_array_equal(inv[order], np.arange(R))
    assert tc.sum() == R and tc.max() <= tile and len(te) <= -(-R // tile) + E
    for e_, o, c in zip(te, to, tc):
        assert np.all(rhs[order[o:o + c]] == e_)
    # ids outside [0, E) sort after every valid route, stably, in tiles of expert -1
    rhs2 = rhs.copy()
    rhs2[[3, 9, 40]] = [-2, E, E + 5]
    order, inv, counts, offsets, te, to, tc = ops.route_plan(rhs2, E, tile)
    assert order[-3:].tolist() == [3, 9, 40]
    assert te.tolist()[-1] == -1 and to.tolist()[-1] == R - 3 and tc.tolist()[-1] == 3
    assert counts.sum() == R - 3 and len(te) <= -(-R // tile) + E


def test_fwht_matches_sylvester_hadamard_and_round_trips():
    n = 64
    H = scipy.linalg.hadamard(n) / np.sqrt(n)
    x = np.random.default_rng(4).standard_normal((3, n))
    np.testing.assert_allclose(rht.fwht(x), x @ H.T, atol=1e-12)
    s = rht.deterministic_rht_signs(n, seed=7)
    y = rht.apply_rht(x, s)
    np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-12)
    np.testing.assert_allclose(rht.apply_inverse_rht(y, s), x, atol=1e-12)
    assert set(np.unique(s).tolist()) <= {-1, 1}


def test_f32_hadamard_restatement_pins():
    # float32 restatement of _hadamard_np against the float64 Sylvester FWHT
    rng = np.random.default_rng(11)
    for n in (16, 128, 4096):
        x = rng.standard_normal((3, n)).astype(np.float32)
        y32 = rht.hadamard_f32(x)
        assert y32.dtype == np.float32
        np.testing.assert_allclose(y32, rht.fwht(x), rtol=0, atol=4e-6 * np.log2(n))
        s = rht.deterministic_rht_signs(n, seed=n)
        np.testing.assert_allclose(rht.apply_rht_f32(x, s), rht.apply_rht(x, s), rtol=0, atol=4e-6 * np.log2(n))
        np.testing.assert_allclose(rht.apply_inverse_rht_f32(rht.apply_rht_f32(x, s), s), x, rtol=0, atol=1e-5)
    # small integers: every butterfly and the power-of-two scale are exact in float32
    n = 256
    xi = rng.integers(-8, 8, size=(2, n)).astype(np.float32)
    H = scipy.linalg.hadamard(n).astype(np.float64) / 16.0
    np.testing.assert_array_equal(rht.hadamard_f32(xi).astype(np.float64), xi.astype(np.float64) @ H.T)


# FIPS 202 SHAKE256 known answer for the empty message (the first 16 output
# bytes of the published test vector).
SHAKE256_EMPTY = bytes.fromhex("46b9dd2b0ba88d13233b3feb743eeb24")
# deterministic_rht_signs(16, seed="") derived by hand from that vector:
# 0x46 = 0100 0110 and 0xb9 = 1011 1001, bits taken least significant first,
# bit 0 -> -1 and bit 1 -> +1.
SIGNS_EMPTY_16 = [-1, 1, 1, -1, -1, -1, 1, -1, 1, -1, -1, 1, 1, 1, -1, 1]


@pytest.mark.parametrize("mod", ["oracle", "product"])
def test_rht_signs_known_answer(mod):
    import hashlib

    from keep_amd import rht as krht
    f = rht.deterministic_rht_signs if mod == "oracle" else krht.deterministic_rht_signs
    assert hashlib.shake_256(b"").digest(16) == SHAKE256_EMPTY
    got = f(16, seed="")
    assert got.dtype == np.int8
    assert got.tolist() == SIGNS_EMPTY_16
    # longer streams continue the same digest: the first 16 of 128 signs are the same
    assert f(128, seed="")[:16].tolist() == SIGNS_EMPTY_16
    # every later byte of the known answer, least significant bit first
    long = f(128, seed="").tolist()
    for i, byte in enumerate(SHAKE256_EMPTY):
        for b in range(8):
            assert long[8 * i + b] == (1 if (byte >> b) & 1 else -1)
    # the seed enters as str(seed) in UTF-8: an int seed equals its decimal string
    assert f(64, seed=13).tolist() == f(64, seed="13").tolist()
    assert f(64, seed=13).tolist() != f(64, seed=14).tolist()
    with pytest.raises(ValueError):
        f(12, seed=0)


def test_c_oracle_decode_matches_numpy_oracle_everywhere():
    t = e8p.e8p_packed_abs_grid()
    np.testing.assert_array_equal(cpu.decode(np.arange(1 << 16, dtype=np.uint16), t), e8p.e8p_full_grid())


def test_c_oracle_matvec_and_moe_match_dense():
    t = e8p.e8p_packed_abs_grid()
    E, H, I, k = 5, 256, 128, 3
    gate, up, down = _proj(E, I, H, 2, 10), _proj(E, I, H, 2, 11), _proj(E, H, I, 1, 12)
    rng = np.random.default_rng(13)
    x = rng.standard_normal((2, H)).astype(np.float32)
    rhs = np.array([[4, 0, 2], [1, 1, 3]])
    y = cpu.routed_matvec(x, gate[0], gate[1].astype(np.float32), t, rhs.reshape(-1), x_div=k, group_size=H // 2)
    want = ops.gather_token(x, gate[0], gate[1], rhs).reshape(6, I)
    assert ops.max_rel_err(y, want) < 1e-5
    w = rng.random((2, k)).astype(np.float32)
    got = cpu.moe_decode(x, rhs, w, gate, up, down, t, limit=10.0, h_bf16=False)
    want = ops.moe_layer(x, rhs, w, gate, up, down, limit=10.0)
    assert ops.max_rel_err(got, want) < 1e-5
    got = cpu.moe_decode(x, rhs, w, gate, up, down, t, limit=0.0, h_bf16=True)
    want = ops.moe_layer(x, rhs, w, gate, up, down, limit=0.0, h_round="bfloat16")
    assert ops.max_rel_err(got, want) < 1e-5


@pytest.mark.parametrize("rg", [1, 2])
def test_c_oracle_nested_tier_matches_dense(rg):
    """The C oracle's nested tier (8-bit E8 residual on the experts listed in
    hot_of_slot, added before the SwiGLU and before the weighted sum) against
    the float64 dense oracle, with per-row and grouped residual scales."""
    t = e8p.e8p_packed_abs_grid()
    E, H, I, k, nhot = 6, 256, 128, 3, 3
    gate, up, down = _proj(E, I, H, 2, 20), _proj(E, I, H, 2, 21), _proj(E, H, I, 1, 22)
    rng = np.random.default_rng(23)
    hot = np.full(E, ops.NO_RESIDUAL, np.uint32)
    hot[[1, 4, 5]] = [2, 0, 1]

    def res(N, K):
        return (rng.integers(0, 256, (nhot, N, K // 8), dtype=np.uint8),
                (np.exp(rng.normal(0, 0.3, (nhot, N, rg))) * 0.1).astype(np.float16))

    residual = {"gate": res(I, H), "up": res(I, H), "down": res(H, I)}
    x = rng.standard_normal((3, H)).astype(np.float32)
    idx = np.array([[1, 0, 4], [5, 2, 3], [0, 2, 3]], dtype=np.int32)  # the last token is all off the tier
    w = rng.random((3, k)).astype(np.float32)
    for limit, hb in ((7.0, False), (0.0, True)):
        got = cpu.moe_decode_nested(x, idx, w, gate, up, down, t, hot, residual, e8p.e8_1bit_packed(),
                                    limit=limit, h_bf16=hb)
        want = ops.moe_layer(x, idx, w, gate, up, down, limit=limit, h_round="bfloat16" if hb else None,
                             hot_of_slot=hot, residual=residual)
        assert ops.max_rel_err(got, want) < 1e-5
    # off the tier the nested form is the plain one, bit for bit
    plain = cpu.moe_decode(x[2:], idx[2:], w[2:], gate, up, down, t, limit=7.0)
    nested = cpu.moe_decode_nested(x[2:], idx[2:], w[2:], gate, up, down, t, hot, residual, e8p.e8_1bit_packed(),
                                   limit=7.0)
    np.testing.assert_array_equal(plain, nested)


def test_c_oracle_residual_matvec_composes_nested_layer():
    """oracle_routed_matvec8 (the tier's residual projection per route) pinned
    by the nested layer oracle: base + residual gate and up, SwiGLU, base +
    residual down on those h, the weighted sum, equal to moe_decode_nested
    (h unrounded) within fp32 rounding; routes off the tier get zeros."""
    t = e8p.e8p_packed_abs_grid()
    t8 = e8p.e8_1bit_packed()
    E, H, I, k, nhot = 6, 256, 128, 3, 3
    gate, up, down = _proj(E, I, H, 2, 30), _proj(E, I, H, 2, 31), _proj(E, H, I, 1, 32)
    rng = np.random.default_rng(33)
    hot = np.full(E, ops.NO_RESIDUAL, np.uint32)
    hot[[1, 4, 5]] = [2, 0, 1]

    def res(N, K, rg):
        return (rng.integers(0, 256, (nhot, N, K // 8), dtype=np.uint8),
                (np.exp(rng.normal(0, 0.3, (nhot, N, rg))) * 0.1).astype(np.float32))

    residual = {"gate": res(I, H, 2), "up": res(I, H, 2), "down": res(H, I, 1)}
    x = rng.standard_normal((3, H)).astype(np.float32)
    idx = np.array([[1, 0, 4], [5, 2, 3], [0, 2, 3]], dtype=np.int32)
    w = rng.random((3, k)).astype(np.float32)
    flat = idx.reshape(-1)
    rows = np.where(hot[flat] == ops.NO_RESIDUAL, -1, hot[flat].astype(np.int64)).astype(np.int32)
    f32 = lambda p: (p[0], p[1].astype(np.float32))  # noqa: E731

    def proj(v, base, name, K, lhs=None, x_div=1):
        b = cpu.routed_matvec(v, *f32(base), t, flat, lhs, x_div=x_div, group_size=K // base[1].shape[-1])
        rc, rs = residual[name]
        r = cpu.routed_matvec8(v, rc, rs, t8, rows, lhs, x_div=x_div, group_size=K // rs.shape[-1])
        return b, r

    gb, gr = proj(x, gate, "gate", H, x_div=k)
    ub, ur = proj(x, up, "up", H, x_div=k)
    assert not gr[rows < 0].any() and gr[rows >= 0].any()
    g, u = gb + gr, ub + ur
    gc, uc = np.minimum(g, 7.0), np.clip(u, -7.0, 7.0)
    h = (gc / (1.0 + np.exp(-gc.astype(np.float64))) * uc).astype(np.float32)
    db, dr = proj(h, down, "down", I, lhs=np.arange(flat.size, dtype=np.int32))
    got = ((db + dr).reshape(3, k, H) * w[..., None]).sum(1)
    want = cpu.moe_decode_nested(x, idx, w, gate, up, down, t, hot, residual, t8, limit=7.0, h_bf16=False)
    assert ops.max_rel_err(got, want) < 1e-5
