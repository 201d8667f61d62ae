"""Pins the CPU oracle's E8P / E8 codebooks and decoders.

Golden literals come from the reference's own tests (tests/golden/reference_literals.json,
transcribed from tests/test_e8_reference.py:23-84); the rest are brute-force and
lattice checks that a dropped term, a wrong nibble index or sign bit fails.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import e8p

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_literals.json").read_text())


def test_e8p_table_sha_and_endpoints():
    t = e8p.e8p_packed_abs_grid()
    assert t.shape == (256,) and t.dtype == np.uint32
    assert e8p.table_sha256(t) == GOLD["e8p_packed_abs_sha256"]
    assert t[:5].tolist() == GOLD["e8p_packed_first5"]
    assert t[-5:].tolist() == GOLD["e8p_packed_last5"]


def test_e8_1bit_table_sha():
    t = e8p.e8_1bit_packed()
    assert e8p.table_sha256(t) == GOLD["e8_1bit_packed_sha256"]


def test_e8p_golden_decodes():
    codes = np.array(GOLD["e8p_decode_codes"], dtype=np.uint16)
    want = np.array(GOLD["e8p_decode_expected"], dtype=np.float32)
    np.testing.assert_array_equal(e8p.decode_e8p(codes), want)
    np.testing.assert_array_equal(e8p.e8p_full_grid()[codes], want)


def test_e8p_signed_base_rows():
    g = e8p.e8p_abs_grid()
    np.testing.assert_array_equal(g[0], np.array(GOLD["e8p_abs_grid_row0"], dtype=np.float32))
    np.testing.assert_array_equal(g[1], np.array(GOLD["e8p_abs_grid_row1"], dtype=np.float32))


def test_e8_1bit_golden_decodes():
    codes = np.array(GOLD["e8_1bit_codes"], dtype=np.uint8)
    np.testing.assert_array_equal(e8p.decode_e8_1bit(codes), np.array(GOLD["e8_1bit_expected"], dtype=np.float32))
    assert not np.array_equal(e8p.decode_e8_1bit(np.arange(256, dtype=np.uint8)),
                              e8p.decode_e8p(np.arange(256, dtype=np.uint16)))


def test_vectorised_decode_matches_bitwise_scalar_decoder_on_every_codeword():
    full = e8p.e8p_full_grid()
    scalar = np.array([e8p.decode_e8p_scalar(c) for c in range(1 << 16)], dtype=np.float32)
    np.testing.assert_array_equal(full, scalar)


def test_e8p_lattice_invariants():
    q = e8p.decode_e8p_half4(np.arange(1 << 16))  # quarter units
    assert np.all(q % 2 != 0)  # every value is an odd multiple of 1/4
    assert np.abs(q).max() <= 15
    parity = np.array([bin(c & 0xFF).count("1") & 1 for c in range(1 << 16)])
    base = q - np.where(parity == 1, -1, 1)[:, None]  # remove the +-1/4 shift
    assert np.all(base % 2 == 0)
    assert np.all((base // 2).sum(axis=1) % 4 == 0)  # half-integer E8 point: even coordinate sum
    assert len(np.unique(q, axis=0)) == 1 << 16  # 65,536 distinct codewords


def test_decode_weight_matrix_matches_manual_table_and_is_exact():
    rng = np.random.default_rng(20260623)
    codes = rng.integers(0, 256, size=(4, 16), dtype=np.uint8)
    scales = rng.normal(loc=1.0, scale=0.05, size=(4, 2)).astype(np.float32)
    dec = e8p.decode_weight_matrix(codes, scales, code_bits=8)
    manual = (e8p.decode_e8_1bit(codes) * np.repeat(scales, 8, axis=-1)[..., None]).reshape(4, 128)
    np.testing.assert_array_equal(dec, manual)
    # E8P value x fp16 scale is exact in fp32: equals the float64 product
    c16 = rng.integers(0, 1 << 16, size=(8, 64), dtype=np.uint16)
    s16 = np.exp(rng.normal(0, 0.3, size=(8, 4))).astype(np.float16)
    d32 = e8p.decode_weight_matrix(c16, s16, code_bits=16)
    d64 = e8p.decode_weight_matrix(c16, s16, code_bits=16, dtype=np.float64)
    np.testing.assert_array_equal(d32.astype(np.float64), d64)


def test_half2_pairs_layout():
    grid = e8p.e8p_abs_grid()
    pairs = e8p.half2_pairs(grid)
    lo = (pairs & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
    hi = (pairs >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(lo, grid[:, 0::2])
    np.testing.assert_array_equal(hi, grid[:, 1::2])


def test_byte_accounting_literal():
    # 2048 rows x 512 codewords x 2 B + 2048 x 8 groups x 2 B scales (group 512, K=4096)
    assert 2048 * 512 * 2 + 2048 * 8 * 2 == GOLD["bytes_per_projection_per_expert_group512"]


@pytest.mark.parametrize("bad", [np.zeros(255, np.uint32)])
def test_decode_rejects_bad_table_shape(bad):
    with pytest.raises((IndexError, ValueError)):
        e8p.decode_e8p(np.array([0xFFFF], dtype=np.uint16), bad)


def test_pair_packed_keeps_every_value_and_inverts():
    """The residual kernels' table layout (reference e8_1bit_m1.py:25-33 and the
    reference's tests/test_e8_1bit_m1.py:32-36): nibbles k and k + 4 hold dims
    2k and 2k + 1; the device-side inverse restores the packed table."""
    import torch

    from keep_amd import ops as kops

    grid = e8p.decode_e8_1bit(np.arange(256))
    pairs = kops.pair_packed(e8p.e8_1bit_packed())
    nib = lambda p, n: ((p >> (4 * n)) & 0xF).astype(np.float64)  # noqa: E731
    back = np.stack([(nib(pairs, d // 2 if d % 2 == 0 else d // 2 + 4) - 8) / 2 for d in range(8)], axis=1)
    np.testing.assert_array_equal(back, grid)
    t = torch.from_numpy(pairs.view(np.int32).copy())
    np.testing.assert_array_equal(kops._unpaired_table(t).numpy().view(np.uint32), e8p.e8_1bit_packed())
