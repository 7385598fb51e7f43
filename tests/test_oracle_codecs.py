"""Pin the oracle's element codecs against independent implementations.

* E4M3 encode/decode: torch's float8_e4m3fn cast (the conversion the reference's
  quantize_block uses, src/vllm_mach/mxfp8/reconstruct_model.py:48), exhaustively
  over every bf16 bit pattern and on random binary32 values.
* FP6 (E2M3 / E3M2): the OCP MX v1.0 value tables and a brute-force nearest-value
  search with saturation and ties-to-even.
* bf16 rounding: torch's float -> bfloat16 cast.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch


def test_e4m3_encode_matches_torch_on_all_bf16(oracle_mod):
    bits = np.arange(65536, dtype=np.uint16)
    f = oracle_mod.bf16_to_f32(bits)
    L = oracle_mod.lib()
    mine = np.array([L.mxo_f32_to_e4m3(float(v)) for v in f], dtype=np.uint8)
    ref = torch.from_numpy(f.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    finite = np.isfinite(f)
    assert np.array_equal(mine[finite], ref[finite])


def test_e4m3_encode_matches_torch_on_random_f32(oracle_mod):
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(100000) * np.exp2(rng.integers(-20, 10, 100000))).astype(np.float32)
    # exact midpoints between E4M3 neighbours (ties) and the overflow region
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    grid = np.unique(grid[np.isfinite(grid)])
    mids = ((grid[1:] + grid[:-1]) / 2).astype(np.float32)
    v = np.concatenate([v, mids, -mids, np.float32([448, 449, 463.9, 464, 464.1, 479.9, 480, 1e9, 2 ** -10])])
    L = oracle_mod.lib()
    mine = np.array([L.mxo_f32_to_e4m3(float(x)) for x in v], dtype=np.uint8)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(mine, ref)


def test_e4m3_decode_matches_torch(oracle_mod):
    dec = oracle_mod.e4m3_to_f32(np.arange(256, dtype=np.uint8))
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    same = (dec == ref) | (np.isnan(dec) & np.isnan(ref))
    assert same.all()


OCP_E2M3_POS = [0, 0.125, 0.25, 0.375, 0.5, 0.625, 0.75, 0.875,
                1.0, 1.125, 1.25, 1.375, 1.5, 1.625, 1.75, 1.875,
                2.0, 2.25, 2.5, 2.75, 3.0, 3.25, 3.5, 3.75,
                4.0, 4.5, 5.0, 5.5, 6.0, 6.5, 7.0, 7.5]
OCP_E3M2_POS = [0, 0.0625, 0.125, 0.1875, 0.25, 0.3125, 0.375, 0.4375,
                0.5, 0.625, 0.75, 0.875, 1.0, 1.25, 1.5, 1.75,
                2.0, 2.5, 3.0, 3.5, 4.0, 5.0, 6.0, 7.0,
                8.0, 10.0, 12.0, 14.0, 16.0, 20.0, 24.0, 28.0]


@pytest.mark.parametrize("fmt,table", [(2, OCP_E2M3_POS), (3, OCP_E3M2_POS)])
def test_fp6_decode_matches_ocp_table(oracle_mod, fmt, table):
    codes = np.arange(64, dtype=np.uint8)
    dec = oracle_mod.fp6_to_f32(codes, fmt)
    assert dec[:32].tolist() == table
    assert dec[32:].tolist() == [-t for t in table]


def _nearest_fp6(x: float, table) -> int:
    """Brute force: saturate, then nearest magnitude in the table, ties to even code."""
    mag = min(abs(Fraction(x)), Fraction(table[-1]))
    best = None
    for code, t in enumerate(table):
        d = abs(mag - Fraction(t))
        if best is None or d < best[0] or (d == best[0] and code % 2 == 0):
            best = (d, code)
    sign = 32 if np.signbit(x) else 0
    return sign | best[1]


@pytest.mark.parametrize("fmt,table", [(2, OCP_E2M3_POS), (3, OCP_E3M2_POS)])
def test_fp6_encode_is_nearest_with_saturation(oracle_mod, fmt, table):
    rng = np.random.default_rng(fmt)
    mids = [(a + b) / 2 for a, b in zip(table[:-1], table[1:])]
    vals = list(rng.uniform(-1.2 * table[-1], 1.2 * table[-1], 3000)) + mids + [-m for m in mids]
    vals += table + [-t for t in table] + [1e-9, -1e-9, 1e6, -1e6]
    L = oracle_mod.lib()
    for v in np.float32(vals):
        got = L.mxo_f32_to_fp6(float(v), fmt)
        want = _nearest_fp6(float(v), table)
        assert got == want, (fmt, float(v), got, want)


def test_fp6_pack_bit_order_and_round_trip(oracle_mod):
    codes = np.array([[1, 2, 3, 4, 63, 0, 62, 5]], dtype=np.uint8)
    packed = oracle_mod.pack_fp6(codes)
    # value i occupies bits [6i, 6i+6) of each little-endian 24-bit group
    w0 = 1 | (2 << 6) | (3 << 12) | (4 << 18)
    w1 = 63 | (0 << 6) | (62 << 12) | (5 << 18)
    assert packed.tolist() == [[w0 & 255, (w0 >> 8) & 255, w0 >> 16, w1 & 255, (w1 >> 8) & 255, w1 >> 16]]
    rng = np.random.default_rng(0)
    c = rng.integers(0, 64, (7, 256)).astype(np.uint8)
    assert np.array_equal(oracle_mod.unpack_fp6(oracle_mod.pack_fp6(c)), c)


def test_bf16_rounding_matches_torch(oracle_mod):
    rng = np.random.default_rng(5)
    v = (rng.standard_normal(50000) * np.exp2(rng.integers(-30, 30, 50000))).astype(np.float32)
    ref = torch.from_numpy(v).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle_mod.f32_to_bf16(v), ref)
    L = oracle_mod.lib()
    assert all(L.mxo_f32_to_bf16(float(x)) == int(r) for x, r in zip(v[:2000], ref[:2000]))


def test_exp_is_accurate(oracle_mod):
    """A wrong reduction constant or polynomial coefficient shows up as > 2 ulp error."""
    x = np.linspace(-87, 88, 20001, dtype=np.float32)
    got = oracle_mod.exp_f32(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 2.0
    assert oracle_mod.exp_f32(np.float32([-88.0, -200.0]))[0] == 0.0
    assert np.isinf(oracle_mod.exp_f32(np.float32([89.0]))[0])
