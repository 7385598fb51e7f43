"""GPU parity: quantizers and producers are bit-exact against the CPU oracle.

Shapes and magnitude sweeps follow the reference's GPU checks
(tests/test_mxfp8_swiglu_quant.py:86-109: M in {1,4,16,24,32,64}, K in {6144,9216},
magnitudes [1, 0, 1e-15, 50]; tests/test_fp8_activation_gpu.py:51-64: rows, seed 1729+rows).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def _inputs(M, K, magnitude, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g) * magnitude
    if outliers and K >= 100:
        x[:, torch.randperm(K, generator=g)[: max(1, K // 100)]] *= 20
    return x.bfloat16()


@pytest.mark.parametrize("rule", [0, 1])
@pytest.mark.parametrize("M,K", [(1, 32), (7, 128), (16, 2048), (33, 5120), (130, 2560)])
@pytest.mark.parametrize("magnitude", [1.0, 0.0, 1e-15, 50.0])
def test_quantize_mxfp8_bit_exact(pkg, oracle_mod, dev, rule, M, K, magnitude):
    x = _inputs(M, K, magnitude, 29 + M + K)
    codes, scales = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), rule)
    rc, rs = oracle_mod.quant_mxfp8(x, rule)
    assert np.array_equal(_u8(scales), rs)
    assert np.array_equal(_u8(codes), rc)


def test_quantize_mxfp8_strided_rows(pkg, oracle_mod, dev):
    base = _inputs(12, 1024, 1.0, 3)
    x = base.to(dev)[:, 256:768]  # row stride 1024, K = 512
    codes, scales = torch.ops.mach_amd.quantize_mxfp8(x, 0)
    rc, rs = oracle_mod.quant_mxfp8(base[:, 256:768].contiguous(), 0)
    assert np.array_equal(_u8(codes), rc) and np.array_equal(_u8(scales), rs)


@pytest.mark.parametrize("M", [1, 4, 16, 24, 32, 64, 128, 512])  # 128 and 512: the c2 prefill producers
@pytest.mark.parametrize("K", [6144, 9216])
def test_swiglu_mxfp8_bit_exact(pkg, oracle_mod, dev, M, K):
    for magnitude in [1.0, 0.0, 1e-15, 50.0]:
        gu = _inputs(M, 2 * K, magnitude, 71 + M, outliers=False)
        codes, scales = torch.ops.mach_amd.swiglu_mxfp8(gu.to(dev), 1, False)
        rc, rs = oracle_mod.swiglu_mxfp8(gu, 1)
        assert np.array_equal(_u8(codes), rc), magnitude
        assert np.array_equal(_u8(scales), rs), magnitude


@pytest.mark.parametrize("M,K", [(1, 9216), (130, 6144), (200, 128), (600, 6144)])  # 600: the table path
def test_swiglu_mxfp8_swizzled_layout(pkg, oracle_mod, dev, M, K):
    gu = _inputs(M, 2 * K, 1.0, 5, outliers=False)
    codes, scales = torch.ops.mach_amd.swiglu_mxfp8(gu.to(dev), 1, True)
    rc, rs = oracle_mod.swiglu_mxfp8(gu, 1)
    assert np.array_equal(_u8(codes), rc)
    assert np.array_equal(_u8(scales), oracle_mod.swizzle_scales(rs, K))


def test_swiglu_rule_floor_carry175(pkg, oracle_mod, dev):
    gu = _inputs(16, 2 * 2048, 3.0, 9, outliers=False)
    codes, scales = torch.ops.mach_amd.swiglu_mxfp8(gu.to(dev), 0, False)
    rc, rs = oracle_mod.swiglu_mxfp8(gu, 0)
    assert np.array_equal(_u8(codes), rc) and np.array_equal(_u8(scales), rs)


@pytest.mark.parametrize("M,K", [(1, 2560), (9, 4096), (512, 2560)])
def test_quantize_block_fp8_bit_exact(pkg, oracle_mod, dev, M, K):
    x = _inputs(M, K, 1.0, 173 + M + K)
    x[0, :128] = 0
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    rq, rsc = oracle_mod.quant_block_fp8(x)
    assert s.stride() == (1, M) or M == 1
    assert np.array_equal(_u8(q), rq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), np.ascontiguousarray(rsc).view(np.uint32))


@pytest.mark.parametrize("rows", [1, 7, 128, 2048])
@pytest.mark.parametrize("transposed", [False, True])
def test_silu_mul_block_fp8_bit_exact(pkg, oracle_mod, dev, rows, transposed):
    g = torch.Generator().manual_seed(1729 + rows)
    x = (torch.randn(rows, 18432, generator=g) * 3).bfloat16()
    out = torch.empty(rows, 9216, dtype=torch.float8_e4m3fn, device=dev)
    if transposed:
        scales = torch.empty(72, rows, dtype=torch.float32, device=dev).t()
    else:
        scales = torch.empty(rows, 72, dtype=torch.float32, device=dev)
    torch.ops.mach_amd.silu_and_mul_per_block_quant(out, x.to(dev), scales, transposed)
    rq, rs = oracle_mod.silu_mul_block_fp8(x, transposed)
    assert np.array_equal(_u8(out), rq)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), np.ascontiguousarray(rs).view(np.uint32))


@pytest.mark.parametrize("fmt", [2, 3])
@pytest.mark.parametrize("M,K,std", [(1, 32, 1.0), (17, 512, 0.015), (256, 5120, 0.015)])
def test_quantize_mxfp6_bit_exact(pkg, oracle_mod, dev, fmt, M, K, std):
    g = torch.Generator().manual_seed(17 + M)
    w = (torch.randn(M, K, generator=g) * std).bfloat16()
    w[0, :32] = 0  # an all-zero block
    packed, scales = torch.ops.mach_amd.quantize_mxfp6(w.to(dev), fmt)
    rc, rs = oracle_mod.quant_mxfp6(w, fmt)
    assert np.array_equal(scales.cpu().numpy(), rs)
    assert np.array_equal(packed.cpu().numpy(), oracle_mod.pack_fp6(rc))


# ---------------------------------------------------------- every bf16 input

def _every_bf16(rows, K, seed=None):
    """All 65536 bf16 bit patterns once -- signed zeros, subnormals, infinities and
    NaNs of both signs and many payloads -- row-major, in order (so blocks mix
    infinities with NaNs) or in a seeded random order."""
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    if seed is not None:
        pats = pats[np.random.default_rng(seed).permutation(65536)]
    assert rows * K == 65536
    return torch.from_numpy(pats.view(np.int16).copy()).view(torch.bfloat16).reshape(rows, K)


@pytest.mark.parametrize("rule", [0, 1, 2])
@pytest.mark.parametrize("seed", [None, 11])
def test_quantize_mxfp8_every_bf16(pkg, oracle_mod, dev, rule, seed):
    x = _every_bf16(8, 8192, seed)
    codes, scales = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), rule)
    rc, rs = oracle_mod.quant_mxfp8(x, rule)
    assert np.array_equal(_u8(scales), rs)
    assert np.array_equal(_u8(codes), rc)
    hi, shi, res, sres = torch.ops.mach_amd.quantize_mxfp8_dual(x.to(dev), rule)
    oh, osh, ores, osres = oracle_mod.quant_mxfp8_dual(x, rule)
    for got, want in ((hi, oh), (shi, osh), (res, ores), (sres, osres)):
        assert np.array_equal(_u8(got), want)


def _every_value_at_every_scale():
    """Blocks that put every bf16 value x with |x| <= A beside a block maximum A, for one
    A per exponent field 0..254 (mantissa 0x5F: the largest before rule 0's carry; the
    sign alternating by exponent): every (value, E8M0 scale) pair the blocks' amax
    reaches, both signs, subnormals and zeros, including the tiny maxima whose rule-0
    scale wraps to 255.  [8411, 1024] bf16."""
    blocks = []
    for e in range(255):
        a = (e << 7) | 0x5F
        mags = np.arange(a + 1, dtype=np.uint32)
        xs = np.concatenate([mags, mags | 0x8000]).astype(np.uint16)
        xs = np.concatenate([xs, np.zeros((-len(xs)) % 31, np.uint16)]).reshape(-1, 31)
        lead = np.full((len(xs), 1), a | ((e & 1) << 15), np.uint16)
        blocks.append(np.concatenate([lead, xs], axis=1))
    b = np.concatenate(blocks)
    b = np.concatenate([b, np.zeros(((-len(b)) % 32, 32), np.uint16)])
    return torch.from_numpy(b.reshape(-1, 1024).view(np.int16).copy()).view(torch.bfloat16)


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_quantize_mxfp8_every_value_at_every_scale(pkg, oracle_mod, dev, rule):
    # the quantizer codes power-of-two-scaled blocks straight from the bf16 pairs (one
    # scaled conversion per pair) and the others with binary32 arithmetic: both against
    # the oracle on every (value, scale) pair
    x = _every_value_at_every_scale()
    codes, scales = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), rule)
    rc, rs = oracle_mod.quant_mxfp8(x, rule)
    assert np.array_equal(_u8(scales), rs)
    assert np.array_equal(_u8(codes), rc)
    assert len(np.unique(rs)) >= (200 if rule == 0 else 100)


@pytest.mark.parametrize("rule", [0, 1, 2])
@pytest.mark.parametrize("seed", [None, 12])
def test_swiglu_mxfp8_every_bf16(pkg, oracle_mod, dev, rule, seed):
    """Every bf16 pattern as gate (up ~ N(0,1)) and as up (gate ~ N(0,1))."""
    pats = _every_bf16(8, 8192, seed)
    other = _inputs(8, 8192, 1.0, 99, outliers=False)
    for gu in (torch.cat([pats, other], dim=1), torch.cat([other, pats], dim=1)):
        codes, scales = torch.ops.mach_amd.swiglu_mxfp8(gu.to(dev), rule, False)
        rc, rs = oracle_mod.swiglu_mxfp8(gu, rule)
        assert np.array_equal(_u8(scales), rs)
        assert np.array_equal(_u8(codes), rc)


@pytest.mark.parametrize("rule", [0, 1])
def test_swiglu_mxfp8_table_every_gate(pkg, oracle_mod, dev, rule):
    """Launches large enough for the producer's SiLU table (2^-24 <= |g| < 256, both signs;
    512 items per CU and up), with only such gates: every one of them in every row, up values
    random, with outliers, infinities and NaNs, so the table path and its quantization
    fallbacks both run; then the same rows with one out-of-range gate per row, which sends
    those waves to the arithmetic."""
    lo, span = 103 << 7, 32 << 7
    gates = np.concatenate([np.arange(lo, lo + span), np.arange(lo, lo + span) | 0x8000]).astype(np.uint16)
    rows = 128
    g = np.stack([np.roll(gates, 97 * r) for r in range(rows)])
    gate = torch.from_numpy(g.view(np.int16).copy()).view(torch.bfloat16)
    up = _inputs(rows, gates.size, 1.0, 77, outliers=True)
    up[1, 5] = float("inf")
    up[2, 9] = float("nan")
    up[3, :32] = 0.0
    for gu in (torch.cat([gate, up], dim=1), torch.cat([gate.clone().index_fill_(1, torch.tensor([300]), 0.0), up], dim=1)):
        assert gu.shape[0] * gu.shape[1] // 2 // 8 >= 512 * 256
        codes, scales = torch.ops.mach_amd.swiglu_mxfp8(gu.to(dev), rule, False)
        rc, rs = oracle_mod.swiglu_mxfp8(gu, rule)
        assert np.array_equal(_u8(scales), rs)
        assert np.array_equal(_u8(codes), rc)


@pytest.mark.parametrize("seed", [None, 13])
def test_block_fp8_producers_every_bf16(pkg, oracle_mod, dev, seed):
    x = _every_bf16(8, 8192, seed)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    rq, rsc = oracle_mod.quant_block_fp8(x)
    assert np.array_equal(_u8(q), rq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), np.ascontiguousarray(rsc).view(np.uint32))
    other = _inputs(8, 8192, 1.0, 98, outliers=False)
    for gu in (torch.cat([x, other], dim=1), torch.cat([other, x], dim=1)):
        out = torch.empty(8, 8192, dtype=torch.float8_e4m3fn, device=dev)
        scales = torch.empty(8, 64, dtype=torch.float32, device=dev)
        torch.ops.mach_amd.silu_and_mul_per_block_quant(out, gu.to(dev), scales, False)
        rq, rs = oracle_mod.silu_mul_block_fp8(gu, False)
        assert np.array_equal(_u8(out), rq)
        assert np.array_equal(scales.cpu().numpy().view(np.uint32), np.ascontiguousarray(rs).view(np.uint32))


@pytest.mark.parametrize("fmt", [2, 3])
@pytest.mark.parametrize("seed", [None, 14])
def test_quantize_mxfp6_every_bf16(pkg, oracle_mod, dev, fmt, seed):
    """Weights are finite: the two infinity patterns are zeroed (the scale of a block
    with an infinite amax is left unspecified); NaNs, subnormals and signed zeros stay."""
    w = _every_bf16(8, 8192, seed)
    w[torch.isinf(w)] = 0
    packed, scales = torch.ops.mach_amd.quantize_mxfp6(w.to(dev), fmt)
    rc, rs = oracle_mod.quant_mxfp6(w, fmt)
    assert np.array_equal(scales.cpu().numpy(), rs)
    assert np.array_equal(packed.cpu().numpy(), oracle_mod.pack_fp6(rc))


# ------------------------------------- champion producer (rp_ue8m0, one rounding)

def _champion_expected(oracle_mod, x):
    codes, scales = oracle_mod.swiglu_mxfp8(x.cpu(), oracle_mod.RULE_RP_UE8M0)
    return codes, oracle_mod.swizzle_scales(scales, x.shape[1] // 2)


@pytest.mark.parametrize("k", [6144, 9216])
@pytest.mark.parametrize("m", [1, 4, 16, 24, 32, 64, 128])
def test_champion_swiglu_bit_exact(pkg, oracle_mod, dev, m, k):
    """Shapes and magnitudes of tests/test_mxfp8_swiglu_quant.py:86-109."""
    g = torch.Generator().manual_seed(1000 + m + k)
    for magnitude in [1.0, 0.0, 1e-15, 50.0]:
        x = (torch.randn(m, 2 * k, generator=g) * magnitude).bfloat16()
        codes, scales = pkg.swiglu_quant.quantize(x.to(dev))
        rc, rs = _champion_expected(oracle_mod, x)
        assert np.array_equal(_u8(codes), rc), magnitude
        assert np.array_equal(_u8(scales), rs), magnitude


def test_champion_graph_replay_with_changing_inputs(pkg, oracle_mod, dev):
    """tests/test_mxfp8_swiglu_quant.py:86-109: capture once, refill the input eagerly,
    replay, compare every replay."""
    m, k = 24, 6144
    x = torch.randn(m, 2 * k, device=dev, dtype=torch.bfloat16)
    pkg.swiglu_quant.quantize(x)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        codes, scales = pkg.swiglu_quant.quantize(x)
    for magnitude in [1.0, 0.0, 1e-15, 50.0, 1.0]:
        x.normal_().mul_(magnitude)
        graph.replay()
        torch.cuda.synchronize()
        rc, rs = _champion_expected(oracle_mod, x)
        assert np.array_equal(_u8(codes), rc), magnitude
        assert np.array_equal(_u8(scales), rs), magnitude


def test_champion_contract(pkg, dev):
    """swiglu_quant.py:23-32: unsupported tensors raise; m == 0 and m > 128 return None."""
    q = pkg.swiglu_quant.quantize
    assert q(torch.zeros(0, 12288, device=dev, dtype=torch.bfloat16)) is None
    assert q(torch.zeros(129, 18432, device=dev, dtype=torch.bfloat16)) is None
    for bad in (torch.zeros(4, 4096, device=dev, dtype=torch.bfloat16),
                torch.zeros(4, 12288, device=dev, dtype=torch.float16),
                torch.zeros(12288, 8, device=dev, dtype=torch.bfloat16).t(),
                torch.zeros(4, 12288, dtype=torch.bfloat16)):
        with pytest.raises(RuntimeError):
            q(bad)
    codes, scales = q(torch.ones(3, 12288, device=dev, dtype=torch.bfloat16))
    assert codes.shape == (3, 6144) and codes.dtype == torch.float8_e4m3fn
    assert scales.shape == (128 * 48 * 4,) and scales.dtype == torch.uint8
    assert pkg.swiglu_quant.inspect()["counts"]
