"""E8P (16-bit) and E8 (8-bit) codebooks and decoders -- CPU oracle (test infrastructure).

Restated from the reference's ``src/keep/vq/e8.py``; each function names the
lines it follows. Values are carried in *half units* (an integer ``h`` stands
for ``h / 2``) until the final float conversion, so every intermediate is exact.

Parity pins (``tests/test_oracle_e8p.py``):

- ``e8p_packed_abs_grid``: SHA-256 of the little-endian table and its first
  and last five words, literals from the reference's
  ``tests/test_e8_reference.py:25,33-34``.
- ``decode_e8p``: the six golden codewords of ``tests/test_e8_reference.py:37-52``
  and the signed base rows of ``:55-62``; plus a bit-by-bit brute-force decoder
  (``decode_e8p_scalar``) over all 65,536 codewords and lattice invariants.
- ``e8_1bit_packed`` / ``decode_e8_1bit``: SHA-256 and the seven golden codes of
  ``tests/test_e8_reference.py:26,65-84``.
- ``decode_weight_matrix``: exactness of value x fp16 scale in fp32 and the
  manual table check of ``tests/test_e8_reference.py:109-120``.
"""

from __future__ import annotations

import hashlib
import itertools
from functools import lru_cache

import numpy as np

CODEWORD_DIM = 8

# Output dimension d of an E8P codeword reads packed nibble SHUFFLE[d]
# (reference ``e8.py:22`` / ``common_e8.metal:6-17``).
E8P_SHUFFLE = (0, 4, 1, 5, 2, 6, 3, 7)

# The 29 norm-12 padding rows that complete the 227 low-norm D8-hat rows to a
# 256-entry table, in half units. This is QuIP#'s fixed padding list (the
# codebook format is shared with the reference, ``e8.py:25-58``); every row has
# five 3s and three 1s (sum of squares 48 half-units^2 = 12).
_E8P_PAD_ROWS_HALF = (
    "31113333", "13113333", "11313333", "11133333", "33313311",
    "33313131", "33311331", "33313113", "33311313", "33311133",
    "33133311", "33133131", "33131331", "33133113", "33131313",
    "33131133", "31333311", "31333131", "31331331", "31333113",
    "31331313", "13331133", "13333311", "13333131", "13331331",
    "13333113", "13331313", "11331333", "33113331",
)


def _pack_nibbles(rows_half: np.ndarray) -> np.ndarray:
    """Pack [N, 8] half-unit ints as ``uint32`` with nibble d = value + 8 (``e8.py:88-100``)."""

    rows = np.asarray(rows_half, dtype=np.int64)
    assert rows.ndim == 2 and rows.shape[1] == CODEWORD_DIM
    nib = rows + 8
    assert nib.min() >= 0 and nib.max() <= 15
    out = np.zeros(rows.shape[0], dtype=np.uint64)
    for d in range(CODEWORD_DIM):
        out |= nib[:, d].astype(np.uint64) << np.uint64(4 * d)
    return out.astype(np.uint32)


def _unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """Inverse of :func:`_pack_nibbles`: ``[..., 8]`` half-unit ints (``e8.py:103-108``)."""

    p = np.asarray(packed, dtype=np.uint32).astype(np.int64)
    return np.stack([((p >> (4 * d)) & 0xF) - 8 for d in range(CODEWORD_DIM)], axis=-1)


def e8p_abs_rows_half() -> np.ndarray:
    """The 256 unshuffled absolute rows in half units (``e8.py:111-124``).

    Rows of {1,3,5,7}^8 with sum of squares <= 40 in ``itertools.product``
    order (227 of them), then the 29 padding rows.
    """

    low = [r for r in itertools.product((1, 3, 5, 7), repeat=8) if sum(v * v for v in r) <= 40]
    assert len(low) == 227
    pads = [tuple(int(c) for c in s) for s in _E8P_PAD_ROWS_HALF]
    return np.array(low + pads, dtype=np.int64)


@lru_cache(maxsize=None)
def _e8p_packed_abs_grid_cached() -> bytes:
    rows = e8p_abs_rows_half()
    # Column order [0,2,4,6,1,3,5,7]: packed nibble j holds source column j's entry.
    shuffled = rows[:, [0, 2, 4, 6, 1, 3, 5, 7]].copy()
    # Parity fix (``e8.py:135-137``): when the half-unit row sum is 2 mod 4,
    # negate packed nibble 7.
    fix = (shuffled.sum(axis=1) % 4) == 2
    shuffled[fix, 7] = -shuffled[fix, 7]
    return _pack_nibbles(shuffled).astype("<u4").tobytes()


def e8p_packed_abs_grid() -> np.ndarray:
    """``uint32[256]`` E8P packed absolute table (``e8.py:127-139``)."""

    return np.frombuffer(_e8p_packed_abs_grid_cached(), dtype="<u4").astype(np.uint32)


def table_sha256(table: np.ndarray) -> str:
    return hashlib.sha256(np.asarray(table, dtype="<u4").tobytes()).hexdigest()


def e8_1bit_rows_half() -> np.ndarray:
    """The 256 signed E8 residual rows in half units (``e8.py:145-166``).

    113 integer rows (entries in {-1,0,1}, sum of squares <= 2, even sum; x2 to
    half units), 128 half rows ({-1,1}^8 with sum = 0 mod 4) and 15 pads
    (+-4 half units on one axis; +e0..+e7 then -e0..-e6).
    """

    ints = [tuple(2 * v for v in r) for r in itertools.product((-1, 0, 1), repeat=8)
            if sum(v * v for v in r) <= 2 and sum(r) % 2 == 0]
    halves = [r for r in itertools.product((-1, 1), repeat=8) if sum(r) % 4 == 0]
    pads = []
    for sign in (4, -4):
        for axis in range(8):
            if sign < 0 and axis == 7:
                break
            row = [0] * 8
            row[axis] = sign
            pads.append(tuple(row))
    rows = np.array(ints + halves + pads, dtype=np.int64)
    assert rows.shape == (256, 8)
    return rows


def e8_1bit_packed() -> np.ndarray:
    """``uint32[256]`` packed E8 residual table (``e8.py:169-179``)."""

    return _pack_nibbles(e8_1bit_rows_half())


def decode_e8_1bit(codes: np.ndarray, table: np.ndarray | None = None) -> np.ndarray:
    """8-bit E8 codes -> float32 ``[..., 8]`` (``e8.py:192-200``)."""

    t = e8_1bit_packed() if table is None else np.asarray(table, dtype=np.uint32)
    c = np.asarray(codes, dtype=np.uint8)
    return (_unpack_nibbles(t[c]).astype(np.float32) * np.float32(0.5))


def decode_e8p_half4(codes: np.ndarray, table: np.ndarray | None = None) -> np.ndarray:
    """E8P codewords -> decoded values in *quarter* units, int64 ``[..., 8]``.

    Follows ``decode_e8p`` (``e8.py:203-234``): ``signs = c & 0xFF``,
    ``idx = c >> 8``, ``p = popcount(signs) & 1``, ``eff = signs ^ p``;
    dim d reads nibble ``s = SHUFFLE[d]``, value ``(nib_s - 8)/2`` negated when
    bit ``s`` of ``eff`` is set, then ``+1/4`` (p = 0) or ``-1/4`` (p = 1).
    Quarter units keep the result integral: value = q / 4.
    """

    t = e8p_packed_abs_grid() if table is None else np.asarray(table, dtype=np.uint32)
    c = np.asarray(codes, dtype=np.uint16).astype(np.int64)
    signs = c & 0xFF
    idx = c >> 8
    parity = np.zeros_like(signs)
    for b in range(8):
        parity ^= (signs >> b) & 1
    eff = signs ^ parity
    half = _unpack_nibbles(t[idx])  # [..., 8] in nibble order
    out = np.empty(c.shape + (8,), dtype=np.int64)
    for d, s in enumerate(E8P_SHUFFLE):
        v = 2 * half[..., s]  # quarter units
        neg = ((eff >> s) & 1).astype(bool)
        out[..., d] = np.where(neg, -v, v) + np.where(parity.astype(bool), -1, 1)
    return out


def decode_e8p(codes: np.ndarray, table: np.ndarray | None = None) -> np.ndarray:
    """E8P codewords -> float32 ``[..., 8]`` (``e8.py:210-234``)."""

    return decode_e8p_half4(codes, table).astype(np.float32) * np.float32(0.25)


def decode_e8p_scalar(code: int) -> list[float]:
    """One codeword decoded bit by bit, written independently of the vectorised
    form (used by the brute-force check over all 65,536 codewords)."""

    table = e8p_packed_abs_grid()
    signs, idx = code & 0xFF, code >> 8
    p = bin(signs).count("1") % 2
    eff = signs ^ p
    word = int(table[idx])
    vals = []
    for d in range(8):
        s = E8P_SHUFFLE[d]
        mag = ((word >> (4 * s)) & 0xF) - 8
        v = mag / 2.0
        if (eff >> s) & 1:
            v = -v
        vals.append(v + (-0.25 if p else 0.25))
    return vals


@lru_cache(maxsize=None)
def _full_grid_bytes() -> bytes:
    return decode_e8p(np.arange(1 << 16, dtype=np.uint16)).tobytes()


def e8p_full_grid() -> np.ndarray:
    """All 65,536 codewords decoded, float32 ``[65536, 8]`` (``e8.py:237-241``)."""

    return np.frombuffer(_full_grid_bytes(), dtype=np.float32).reshape(65536, 8).copy()


def e8p_abs_grid() -> np.ndarray:
    """Signed base rows in output-dimension order, float32 ``[256, 8]`` (``e8.py:244-252``)."""

    half = _unpack_nibbles(e8p_packed_abs_grid())
    return half[:, list(E8P_SHUFFLE)].astype(np.float32) * np.float32(0.5)


def decode_weight_matrix(codes: np.ndarray, scales: np.ndarray | None = None, *, code_bits: int = 16,
                         table: np.ndarray | None = None, dtype=np.float32) -> np.ndarray:
    """Dense dequantisation ``[..., C] -> [..., 8*C]`` (``e8.py:542-571``).

    ``scales[..., G]`` partitions the C codewords of a row into G equal groups.
    The product value x scale is computed in ``dtype`` (float32 by default, as
    the reference; every E8P value times an fp16 scale is exact in float32).
    """

    if code_bits == 16:
        dec = decode_e8p(codes, table)
    elif code_bits == 8:
        dec = decode_e8_1bit(codes, table)
    else:
        raise ValueError("code_bits must be 8 or 16")
    dec = dec.astype(dtype)
    if scales is not None:
        sc = np.asarray(scales).astype(dtype)
        C = dec.shape[-2]
        if C % sc.shape[-1]:
            raise ValueError("codeword count must be divisible by scale count")
        dec = dec * np.repeat(sc, C // sc.shape[-1], axis=-1)[..., None]
    return dec.reshape(dec.shape[:-2] + (dec.shape[-2] * CODEWORD_DIM,))


def half2_pairs(grid: np.ndarray) -> np.ndarray:
    """``[256, 8]`` exact-in-fp16 codebook -> ``uint32[256, 4]`` with entry k =
    fp16 bits of dim 2k (low half) and 2k+1 (high half)
    (reference ``src/ramp/kernels/e8p_nested_m1.py:29-36``)."""

    h = np.asarray(grid).astype(np.float16)
    assert h.shape == (256, 8) and np.array_equal(h.astype(np.float64), np.asarray(grid, dtype=np.float64))
    bits = h.view(np.uint16).astype(np.uint32)
    return np.ascontiguousarray(bits[:, 0::2] | (bits[:, 1::2] << 16))
