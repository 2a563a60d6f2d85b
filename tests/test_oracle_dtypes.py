"""Pins the oracle's raw-cache conversions (orc_f32_to_f16, orc_f32_to_bf16 and their
upcasts; src/engine/io/gguf.rs:26-117) that every f16/bf16 prefill parity test uses to
round the K/V rows it writes into the cache (CPU only).

Independent checks: numpy's IEEE half conversion, torch's bf16 conversion, and a
float64 nearest-value search over the full f16 / bf16 grids with ties to the even
pattern; exhaustive over all 65,536 patterns for the upcasts.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch


def _edge_f32_bits() -> np.ndarray:
    """Ties, subnormals, the overflow boundary, zeros, infinities and NaNs."""
    e = []
    # f16: exact halfway points between neighbours in the normal range (mantissa
    # bit 12 set, bits 0..11 clear) with both parities of the kept mantissa, and
    # one ulp either side of each.
    for exp in (103, 112, 113, 120, 127, 135, 142):
        for man in (0x000000, 0x001000, 0x003000, 0x7fe000, 0x7ff000, 0x400000 | 0x1000,
                    0x400000 | 0x3000):
            b = (exp << 23) | man
            e += [b - 1, b, b + 1]
    # Subnormal f16 range: 2^-25 (half the smallest subnormal, ties to 0), 2^-24,
    # 1.5 * 2^-24 (tie, rounds to even 2^-23), 2^-14 minus one f32 ulp.
    e += [0x33000000, 0x33000001, 0x32ffffff, 0x33800000, 0x33c00000, 0x34400000, 0x387fffff,
          0x38800000, 0x387fe000, 0x387ff000]
    # Overflow boundary: 65504 (max f16), 65519.99 (rounds down), 65520 (ties up to inf).
    e += [0x477fe000, 0x477fefff, 0x477ff000, 0x477ff001, 0x47800000, 0x7f7fffff]
    # bf16 ties: low 16 bits exactly 0x8000 with even / odd kept bits.
    e += [0x3f808000, 0x3f818000, 0x3f807fff, 0x3f808001, 0x7f7f8000, 0x7f7fffff, 0x00008000,
          0x00018000]
    # Zeros, f32 subnormals, infinities, quiet and signalling NaNs.
    e += [0x00000000, 0x00000001, 0x007fffff, 0x7f800000, 0x7fc00000, 0x7fc00001, 0x7fffffff,
          0x7f800001, 0x7fa00000, 0x7f802000, 0x7fbfe000]
    b = np.array(e, np.uint32)
    return np.concatenate([b, b | 0x80000000]).astype(np.uint32)


@pytest.fixture(scope="module")
def f32_patterns() -> np.ndarray:
    rng = np.random.default_rng(20260)
    rand_bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # Values concentrated near the f16 range so its rounding paths get most of them.
    near = rng.integers(0x30000000, 0x48000000, size=100_000, dtype=np.uint64).astype(np.uint32)
    near |= (rng.integers(0, 2, size=near.size) << 31).astype(np.uint32)
    return np.concatenate([_edge_f32_bits(), rand_bits, near])


def _is_nan_bits32(b):
    return (b & 0x7FFFFFFF) > 0x7F800000


def _nearest_even(x64: np.ndarray, grid_bits: np.ndarray, grid_vals: np.ndarray) -> np.ndarray:
    """Pattern of the grid value nearest to x64 (ties to the even pattern), grids of
    finite non-negative values sorted ascending; magnitudes only."""
    ax = np.abs(x64)
    hi = np.searchsorted(grid_vals, ax, side="left")
    hi = np.minimum(hi, grid_vals.size - 1)
    lo = np.maximum(hi - 1, 0)
    d_lo = ax - grid_vals[lo]
    d_hi = grid_vals[hi] - ax
    take_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((grid_bits[hi] & 1) == 0))
    return np.where(take_hi, grid_bits[hi], grid_bits[lo])


def test_f32_to_f16_matches_numpy(orc, f32_patterns):
    b = f32_patterns
    x = b.view(np.float32)
    got = orc.c_f32_to_f16(x)
    with np.errstate(over="ignore"):
        exp = x.astype(np.float16).view(np.uint16)
    nan = _is_nan_bits32(b)
    quiet = nan & ((b & 0x00400000) != 0)
    # numpy keeps a quiet NaN's payload exactly as the reference (top mantissa bits).
    ok = ~nan | quiet
    assert np.array_equal(got[ok], exp[ok]), np.flatnonzero(got[ok] != exp[ok])[:10]
    # Signalling NaNs: a NaN of the same sign, quieted, with the top 9 payload bits kept.
    g = got[nan & ~quiet]
    s = b[nan & ~quiet]
    assert np.all((g & 0x7C00) == 0x7C00) and np.all((g & 0x3FF) != 0)
    assert np.all((g & 0x200) != 0)
    assert np.array_equal(g & 0x1FF, ((s >> 13) & 0x1FF).astype(np.uint16))
    assert np.array_equal(g >> 15, (s >> 31).astype(np.uint16))


def test_f32_to_f16_nearest_even_float64(orc, f32_patterns):
    """Round to nearest (ties to even) on the exact f16 value grid; |x| >= 65520 -> inf."""
    b = f32_patterns[~_is_nan_bits32(f32_patterns)]
    x = b.view(np.float32)
    got = orc.c_f32_to_f16(x)
    grid_bits = np.arange(0, 0x7C00, dtype=np.uint16)
    grid_vals = grid_bits.view(np.float16).astype(np.float64)
    x64 = x.astype(np.float64)
    mag = _nearest_even(x64, grid_bits, grid_vals)
    mag = np.where(np.abs(x64) >= 65520.0, np.uint16(0x7C00), mag).astype(np.uint16)
    exp = mag | ((b >> 16) & 0x8000).astype(np.uint16)
    assert np.array_equal(got, exp), np.flatnonzero(got != exp)[:10]


def test_f32_to_f16_named_cases(orc):
    cases = {
        0x477FF000: 0x7C00,  # 65520 ties to the even neighbour, which is inf
        0x477FEFFF: 0x7BFF,  # just below: 65504
        0x33000000: 0x0000,  # 2^-25: tie between 0 and the smallest subnormal -> 0
        0x33000001: 0x0001,
        0x33C00000: 0x0002,  # 1.5 * 2^-24: tie -> even (2 * 2^-24)
        0x3F800000: 0x3C00,  # 1.0
        0x3F801000: 0x3C00,  # 1 + 2^-11: tie -> even (1.0)
        0x3F803000: 0x3C02,  # 1 + 3 * 2^-11: tie -> even (1 + 2^-9)
        0xFF800000: 0xFC00,
        0x7FC00000: 0x7E00,
    }
    b = np.array(list(cases), np.uint32)
    got = orc.c_f32_to_f16(b.view(np.float32))
    assert [int(v) for v in got] == list(cases.values())


def test_f32_to_bf16_matches_torch_and_float64(orc, f32_patterns):
    b = f32_patterns
    x = b.view(np.float32)
    got = orc.c_f32_to_bf16(x)
    nan = _is_nan_bits32(b)
    exp_t = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[~nan], exp_t[~nan]), np.flatnonzero(got[~nan] != exp_t[~nan])[:10]
    # float64 nearest-even on the bf16 grid; beyond the largest finite bf16 plus half
    # an ulp (2^128 - 2^119) the result is inf.
    grid_bits = np.arange(0, 0x7F80, dtype=np.uint16)
    grid_vals = (grid_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    fin = ~nan & ((b & 0x7FFFFFFF) < 0x7F800000)
    x64 = x[fin].astype(np.float64)
    mag = _nearest_even(x64, grid_bits, grid_vals)
    mag = np.where(np.abs(x64) >= 2.0**128 - 2.0**119, np.uint16(0x7F80), mag).astype(np.uint16)
    exp64 = mag | ((b[fin] >> 16) & 0x8000).astype(np.uint16)
    assert np.array_equal(got[fin], exp64), np.flatnonzero(got[fin] != exp64)[:10]
    # NaNs stay NaN (never inf), sign and top payload bits kept, quiet bit forced.
    g = got[nan]
    assert np.all((g & 0x7F80) == 0x7F80) and np.all((g & 0x7F) != 0)
    assert np.all((g & 0x40) != 0)
    assert np.array_equal(g & 0xFFBF, ((b[nan] >> 16) & 0xFFBF).astype(np.uint16))


def test_numpy_bf16_bits_helper_matches_oracle(orc, f32_patterns):
    """The tests' input rounding helper (oracle.py bf16_bits) is the same rounding."""
    x = f32_patterns.view(np.float32)
    assert np.array_equal(orc.bf16_bits(x), orc.c_f32_to_bf16(x))
    nan = _is_nan_bits32(f32_patterns)
    with np.errstate(over="ignore"):
        assert np.array_equal(orc.f16_bits(x)[~nan], orc.c_f32_to_f16(x)[~nan])


def test_f16_to_f32_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.c_f16_to_f32(h).view(np.uint32)
    nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    exp = h.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got[~nan], exp[~nan]), np.flatnonzero(got[~nan] != exp[~nan])[:10]
    # NaN payloads widen bit for bit: sign, all-ones exponent, payload << 13.
    hn = h[nan].astype(np.uint32)
    assert np.array_equal(got[nan], ((hn & 0x8000) << 16) | 0x7F800000 | ((hn & 0x3FF) << 13))
    # Exact: every finite half survives the round trip through the oracle's downcast.
    fin = (h & 0x7C00) != 0x7C00
    back = orc.c_f32_to_f16(got[fin].view(np.float32))
    assert np.array_equal(back, h[fin])


def test_bf16_to_f32_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.c_bf16_to_f32(h).view(np.uint32)
    exp = torch.from_numpy(h.view(np.int16).copy()).view(torch.bfloat16).float().numpy().view(np.uint32)
    nan = ((h & 0x7F80) == 0x7F80) & ((h & 0x7F) != 0)
    assert np.array_equal(got[~nan], exp[~nan])
    assert np.array_equal(got, h.astype(np.uint32) << 16)
    fin = (h & 0x7F80) != 0x7F80
    assert np.array_equal(orc.c_f32_to_bf16(got[fin].view(np.float32)), h[fin])
