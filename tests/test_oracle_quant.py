"""Pin the oracle's quantizers and producers.

* floor_carry175 (quantize_block, src/vllm_mach/mxfp8/reconstruct_model.py:34-50):
  the reference's stored known answer (tests/golden/mxfp8_quantize_block_kat.json)
  and codes/scales from the reference's own torch arithmetic (log2 / floor / exp2 /
  float8 cast), a different primitive path than the oracle's bit operations.
* ceil_div448 (mxfp6/mxfp8_mlp.py:100-105): exact rational arithmetic
  (s = ceil(log2(amax / 448)) + 127), the zero-block floor (s = 28), and torch's
  float8 cast for the codes.
* SwiGLU producer wiring (gate/up halves, both bf16 roundings, scale swizzle) and
  block-FP8 quantizers against torch evaluations of the same formulas, plus the
  swizzle's bijectivity and the reference test's own index expression
  (tests/test_mxfp8_swiglu_quant.py:100-102).
"""
import json
import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def _torch_quantize_block(x: torch.Tensor):
    """The reference's arithmetic, evaluated with torch primitives."""
    maximum = x.reshape(x.shape[0], -1, 32).abs().amax(-1)
    bits = maximum.view(torch.uint16).to(torch.int32)
    rounded = ((bits + 32) & 0xFF80).to(torch.uint16).view(torch.bfloat16)
    scales = (127 + torch.floor(torch.log2(rounded)) - 8).to(torch.uint8)
    expanded = torch.exp2(scales.float() - 127).repeat_interleave(32, -1)
    codes = (x.float() / expanded).to(torch.float8_e4m3fn)
    return codes.view(torch.uint8).numpy(), scales.numpy()


def test_floor_carry175_known_answer(oracle_mod):
    kat = json.loads((GOLDEN / "mxfp8_quantize_block_kat.json").read_text())
    x = torch.tensor([[v, -v] * 16 for v in kat["maxima"]], dtype=torch.bfloat16)
    codes, scales = oracle_mod.quant_mxfp8(x, oracle_mod.RULE_FLOOR_CARRY175)
    assert scales.ravel().tolist() == kat["expected_scales"]
    # codes of the known answer: x / 2^(s-127) cast to E4M3 (the test's closed form)
    tc, ts = _torch_quantize_block(x)
    assert np.array_equal(codes, tc)


@pytest.mark.parametrize("magnitude", [1.0, 0.0, 1e-15, 50.0, 3e4])
def test_floor_carry175_matches_reference_arithmetic(oracle_mod, magnitude):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(64, 1024, generator=g) * magnitude
    x[:, torch.randperm(1024, generator=g)[:10]] *= 20  # outlier channels
    x = x.bfloat16()
    codes, scales = oracle_mod.quant_mxfp8(x, oracle_mod.RULE_FLOOR_CARRY175)
    tc, ts = _torch_quantize_block(x)
    assert np.array_equal(scales, ts)
    assert np.array_equal(codes, tc)


def _exact_ceil448_scale(amax: float) -> int:
    raw = Fraction(amax) / 448 if amax > 0 else Fraction(0)
    if raw < Fraction(1e-30):  # the rule's floor, a binary32 literal
        raw = Fraction(float(np.float32(1e-30)))
    e = math.floor(math.log2(raw))
    while Fraction(2) ** e < raw:
        e += 1
    while Fraction(2) ** (e - 1) >= raw:
        e -= 1
    return e + 127


def test_ceil_div448_scales_exact_rational(oracle_mod):
    rng = np.random.default_rng(2)
    amax = np.concatenate([
        rng.standard_normal(200) * np.exp2(rng.integers(-40, 40, 200)),
        np.float32([448, 448 * 2, 448 * 1.5, 0.0, 1.75, 1.7578125, 1.0, 2 ** -100, 7.0, 14.0]),
    ])
    rows = []
    for a in amax:
        row = np.zeros(32, np.float32)
        row[5] = a
        rows.append(row)
    x = torch.from_numpy(np.stack(rows)).bfloat16()
    _, scales = oracle_mod.quant_mxfp8(x, oracle_mod.RULE_CEIL_DIV448)
    amax_bf = x.float().abs().amax(-1).numpy()
    want = [_exact_ceil448_scale(float(a)) for a in amax_bf]
    assert scales.ravel().tolist() == want
    assert want[-7] == 28  # zero block


def test_ceil_div448_codes_match_torch(oracle_mod):
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(32, 512, generator=g) * 3).bfloat16()
    codes, scales = oracle_mod.quant_mxfp8(x, oracle_mod.RULE_CEIL_DIV448)
    inv = torch.exp2(127 - torch.from_numpy(scales).float()).repeat_interleave(32, -1)
    ref = (x.float() * inv).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, ref)
    assert (np.abs(x.float().numpy() * inv.numpy()) <= 448).all()


def test_swiglu_producer_wiring(oracle_mod):
    g = torch.Generator().manual_seed(71)
    M, K = 6, 256
    gu = (torch.randn(M, 2 * K, generator=g) * 2).bfloat16()
    codes, scales = oracle_mod.swiglu_mxfp8(gu, oracle_mod.RULE_CEIL_DIV448)
    gate, up = gu[:, :K].float(), gu[:, K:].float()
    e = torch.from_numpy(oracle_mod.exp_f32((-gate).numpy()))
    act = (gate / (1.0 + e)).bfloat16().float()
    v = (act * up).bfloat16()
    c2, s2 = oracle_mod.quant_mxfp8(v, oracle_mod.RULE_CEIL_DIV448)
    assert np.array_equal(codes, c2) and np.array_equal(scales, s2)
    # agreement with torch's own SiLU: the only differences are bf16 tie flips
    v_t = (torch.nn.functional.silu(gate).bfloat16().float() * up).bfloat16()
    c3, _ = oracle_mod.quant_mxfp8(v_t, oracle_mod.RULE_CEIL_DIV448)
    assert (codes == c3).mean() > 0.99


def test_swizzle_is_reference_map_and_bijective(oracle_mod):
    for M, K in [(1, 9216), (130, 6144), (300, 128)]:
        rows = np.arange(M)[:, None]
        groups = np.arange(K // 32)[None, :]
        # index expression of tests/test_mxfp8_swiglu_quant.py:100-102
        ref = (((rows // 128 * ((K // 32 + 3) // 4) + groups // 4) * 32 + rows % 32) * 4 + rows % 128 // 32) * 4 + groups % 4
        logical = np.random.default_rng(M).integers(0, 256, (M, K // 32)).astype(np.uint8)
        flat = oracle_mod.swizzle_scales(logical, K)
        assert flat.size == (M + 127) // 128 * 128 * ((K // 32 + 3) // 4) * 4
        assert np.array_equal(flat[ref], logical)
        assert len(np.unique(ref)) == ref.size


def test_block_fp8_quant_matches_torch(oracle_mod):
    g = torch.Generator().manual_seed(173)
    x = torch.randn(9, 512, generator=g).bfloat16()
    x[3] = 0  # zero rows take the 1e-10 floor
    q, s = oracle_mod.quant_block_fp8(x)
    xf = x.float().reshape(9, 4, 128)
    amax = xf.abs().amax(-1).clamp_min(1e-10)
    scale = amax / 448.0
    ref_q = (xf / scale[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).reshape(9, 512)
    assert np.array_equal(s, scale.numpy())
    assert np.array_equal(q, ref_q.numpy())
    assert not s.flags["C_CONTIGUOUS"]  # column-major data, as the reference stores it


@pytest.mark.parametrize("transposed", [False, True])
def test_silu_mul_block_fp8_matches_torch(oracle_mod, transposed):
    g = torch.Generator().manual_seed(1729)
    rows, H = 5, 256
    x = (torch.randn(rows, 2 * H, generator=g) * 4).bfloat16()
    q, s = oracle_mod.silu_mul_block_fp8(x, transposed)
    gate, up = x[:, :H].float(), x[:, H:].float()
    e = torch.from_numpy(oracle_mod.exp_f32((-gate).numpy()))
    v = (gate * (1.0 / (1.0 + e))) * up
    vg = v.reshape(rows, 2, 128)
    scale = torch.maximum(vg.abs().amax(-1) / 448.0, torch.tensor(1.0 / (448.0 * 512.0)))
    ref_q = (vg / scale[..., None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).reshape(rows, H)
    assert np.array_equal(q, ref_q.numpy())
    assert np.array_equal(np.asarray(s), scale.numpy())


@pytest.mark.parametrize("fmt", [2, 3])
def test_mxfp6_quant_ocp_rule(oracle_mod, fmt):
    """Shared exponent floor(log2 amax) - emax (OCP MX v1.0 section 6.3) and every element
    the saturated nearest grid value of x / 2^exp (brute force over the OCP table)."""
    from test_oracle_codecs import OCP_E2M3_POS, OCP_E3M2_POS, _nearest_fp6
    table = OCP_E2M3_POS if fmt == 2 else OCP_E3M2_POS
    g = torch.Generator().manual_seed(17)
    w = (torch.randn(4, 256, generator=g) * 0.015).bfloat16()
    w[0, :32] = 0  # all-zero block -> code 0
    codes, scales = oracle_mod.quant_mxfp6(w, fmt)
    emax = 2 if fmt == 2 else 4
    amax = w.float().reshape(4, 8, 32).abs().amax(-1).numpy()
    with np.errstate(divide="ignore"):
        want = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1))).astype(int) - emax + 127, 0)
    assert np.array_equal(scales.astype(int), want)
    wf = w.float().numpy()
    for r in range(4):
        for k in range(256):
            x = Fraction(float(wf[r, k])) / Fraction(2) ** (int(scales[r, k // 32]) - 127)
            assert codes[r, k] == _nearest_fp6(float(x), table) | (32 if np.signbit(wf[r, k]) else 0) & 63


# ------------------------------------------------ rp_ue8m0 (champion producer)

def _rp_scale_bruteforce(amax: np.float32) -> int:
    """Smallest E8M0 code s (0..254) with 2^(s-127) >= fl32(amax * fl32(1/448)),
    254 when none is (mxfp8/swiglu_quant.py:58-61, satfinite), by exhaustive search."""
    raw = float(np.float32(np.float32(amax) * (np.float32(1.0) / np.float32(448.0))))
    for s in range(255):
        if Fraction(2) ** (s - 127) >= Fraction(raw):
            return s
    return 254


def test_rp_ue8m0_constant_is_correctly_rounded():
    r = np.float32(1.0) / np.float32(448.0)
    assert r.view(np.uint32) == 0x3B124925
    assert abs(Fraction(float(r)) - Fraction(1, 448)) <= Fraction(1, 2) * Fraction(2) ** -32  # half an ulp


def test_rp_ue8m0_scales_bruteforce(oracle_mod):
    rng = np.random.default_rng(3)
    amax = np.concatenate([
        rng.standard_normal(300) * np.exp2(rng.integers(-130, 120, 300)),
        # exact powers of two times 448 (raw lands on a power of two), the E4M3
        # maximum's neighbours, subnormal raw on both sides of 2^-127, zero, huge
        np.float32([448, 896, 448 * 2.0 ** -20, 447, 449, 1.75, 0.0, 2.0 ** -126,
                    2.0 ** -117, 2.0 ** -118, 3.0e38, 1.0e-38]),
    ])
    rows = np.zeros((amax.size, 32), np.float32)
    rows[:, 7] = amax
    x = torch.from_numpy(rows).bfloat16()
    _, scales = oracle_mod.quant_mxfp8(x, oracle_mod.RULE_RP_UE8M0)
    amax_bf = x.float().abs().amax(-1).numpy()
    assert scales.ravel().tolist() == [_rp_scale_bruteforce(a) for a in amax_bf]
    # raw = 2^k exactly for amax = 448 * 2^k: no round-up (the constant is correctly rounded)
    assert scales[300, 0] == 127 and scales[301, 0] == 128
    assert scales[306, 0] == 0  # zero block


def test_rp_ue8m0_codes_match_torch(oracle_mod):
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(64, 512, generator=g) * torch.exp2(torch.randint(-30, 30, (64, 1), generator=g))).bfloat16()
    x[0] = 0
    codes, scales = oracle_mod.quant_mxfp8(x, oracle_mod.RULE_RP_UE8M0)
    s = torch.from_numpy(scales).float()
    inv = torch.where((s == 0) | (s == 254), torch.zeros_like(s), torch.exp2(127 - s)).repeat_interleave(32, -1)
    ref = (x.float() * inv).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(codes, ref)
    assert (codes[0] == 0).all() and scales[0].tolist() == [0] * 16


def test_rp_ue8m0_special_values(oracle_mod):
    """inf amax saturates the scale at 254, whose inverse is 0 (2^-127 flushed); a NaN
    element is skipped by the amax and, as the clamp max(., -448) comes first, coded -448."""
    row = np.zeros((2, 32), np.float32)
    row[0, 3], row[0, 4] = np.inf, 2.0
    row[1, 3], row[1, 4] = np.nan, 448.0
    codes, scales = oracle_mod.quant_mxfp8(torch.from_numpy(row).bfloat16(), oracle_mod.RULE_RP_UE8M0)
    assert scales[0, 0] == 254 and codes[0, 3] == 0xFE and codes[0, 4] == 0  # inf * 0 = NaN -> -448
    assert scales[1, 0] == 127 and codes[1, 3] == 0xFE and codes[1, 4] == 0x7E


def test_champion_swiglu_is_quantize_of_single_rounded_silu(oracle_mod):
    """The reference test's identity (tests/test_mxfp8_swiglu_quant.py:86-109): the fused
    producer equals the rp_ue8m0 quantizer applied to bf16((g / (1 + exp(-g))) * up)."""
    g = torch.Generator().manual_seed(71)
    M, K = 6, 512
    for magnitude in [1.0, 0.0, 1e-15, 50.0]:
        gu = (torch.randn(M, 2 * K, generator=g) * magnitude).bfloat16()
        codes, scales = oracle_mod.swiglu_mxfp8(gu, oracle_mod.RULE_RP_UE8M0)
        gate, up = gu[:, :K].float(), gu[:, K:].float()
        e = torch.from_numpy(oracle_mod.exp_f32((-gate).numpy()))
        v = ((gate / (1.0 + e)) * up).bfloat16()  # one rounding: no bf16 SiLU
        c2, s2 = oracle_mod.quant_mxfp8(v, oracle_mod.RULE_RP_UE8M0)
        assert np.array_equal(codes, c2) and np.array_equal(scales, s2), magnitude
    # torch's own SiLU composition differs only by exp ulps
    v_t = (torch.nn.functional.silu(gate) * up).bfloat16()
    c3, _ = oracle_mod.quant_mxfp8(v_t, oracle_mod.RULE_RP_UE8M0)
    assert (codes == c3).mean() > 0.99
