"""GPU parity of the residual + Gemma RMSNorm (+ MXFP8) producer against the oracle:
codes, scales (logical and swizzled), the summed residual and the bf16 normalized output
are bit-exact (mxfp6/mxfp8_norm_quant.py:15-39, mxfp6/gemma_norm.py:13-29).  Shapes cover
the smallest and largest admitted N, rows past one 128-row scale tile, no residual, zero
and large rows; the fused norm -> gate_up GEMM meets the GEMM bar."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import _check, _weights

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _case(M, N, seed, residual=True, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, N, generator=g) * scale).bfloat16()
    r = (torch.randn(M, N, generator=g) * 3 * scale).bfloat16() if residual else None
    w = (torch.randn(N, generator=g) * 0.2).bfloat16()
    return x, r, w


@pytest.mark.parametrize("M,N,residual,swizzled,rule", [
    (1, 32, True, True, 1),
    (7, 2560, True, True, 1),
    (130, 5120, True, True, 1),      # two 128-row scale tiles
    (3, 16384, False, False, 1),     # the largest N: eight chunks per thread
    (33, 2048, True, False, 0),      # floor_carry175 scales
    (64, 4096, False, True, 1),
])
def test_rmsnorm_mxfp8_bit_exact(pkg, oracle_mod, dev, M, N, residual, swizzled, rule):
    x, r, w = _case(M, N, 11 + M + N, residual)
    eps = 1e-6
    codes, scales, summed = torch.ops.mach_amd.rmsnorm_mxfp8(
        x.to(dev), r.to(dev) if residual else None, w.to(dev), eps, rule, swizzled)
    rc, rs, rsum = oracle_mod.rmsnorm_mx(x, r, w, eps, rule)
    assert np.array_equal(_u8(codes), rc)
    if swizzled:
        ref = np.zeros(oracle_mod.lib().mxo_swizzle_size(M, N), np.uint8)
        oracle_mod.lib().mxo_swizzle_scales(oracle_mod._p(np.ascontiguousarray(rs)), M, N, oracle_mod._p(ref))
        assert np.array_equal(_u8(scales), ref)
    else:
        assert np.array_equal(_u8(scales), rs)
    if residual:
        assert np.array_equal(_bits(summed), rsum)
    else:
        assert torch.equal(summed.cpu(), x)


def test_rmsnorm_mxfp8_zero_and_large_rows(pkg, oracle_mod, dev):
    x, r, w = _case(4, 1024, 5)
    x[0] = 0.0
    r[0] = 0.0
    x[1] *= 3000.0
    x[2, :512] = 1e-20
    for rule in (0, 1):
        codes, scales, summed = torch.ops.mach_amd.rmsnorm_mxfp8(x.to(dev), r.to(dev), w.to(dev), 1e-5, rule, False)
        rc, rs, rsum = oracle_mod.rmsnorm_mx(x, r, w, 1e-5, rule)
        assert np.array_equal(_u8(codes), rc) and np.array_equal(_u8(scales), rs)
        assert np.array_equal(_bits(summed), rsum)


@pytest.mark.parametrize("M,N,residual", [(1, 256, True), (17, 2560, True), (40, 8192, False)])
def test_gemma_rmsnorm_bit_exact(pkg, oracle_mod, dev, M, N, residual):
    x, r, w = _case(M, N, 3 + M, residual)
    y, summed = torch.ops.mach_amd.gemma_rmsnorm(x.to(dev), r.to(dev) if residual else None, w.to(dev), 1e-6)
    ry, rsum = oracle_mod.rmsnorm_mx(x, r, w, 1e-6, quant=False)
    assert np.array_equal(_bits(y), ry)
    if residual:
        assert np.array_equal(_bits(summed), rsum)
    else:
        assert summed.numel() == 0


def test_rmsnorm_rejects_bad_shapes(pkg, dev):
    x = torch.zeros(2, 48, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        torch.ops.mach_amd.rmsnorm_mxfp8(x, None, torch.zeros(48, dtype=torch.bfloat16, device=dev), 1e-6, 1, True)
    x = torch.zeros(2, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        torch.ops.mach_amd.gemma_rmsnorm(x, x[:1], torch.zeros(64, dtype=torch.bfloat16, device=dev), 1e-6)


@pytest.mark.parametrize("M", [1, 16, 200])
def test_norm_mx_gate_up(pkg, oracle_mod, dev, M):
    """Producer + gate_up GEMM (mach_norm_quant_mxfp8_gate_up, mxfp8_norm_quant.py:58-72)."""
    ops = pkg.ops
    N, K = 1024, 2560
    x, r, nw = _case(M, K, 41 + M)
    wc, ws, stored = _weights(oracle_mod, N, K, 0, 0.02, 5)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), 0)
    y, summed = ops.norm_mx_gate_up(x.to(dev), r.to(dev), nw.to(dev), 1e-6, tiled, tiled_s, N)
    ac, as_, rsum = oracle_mod.rmsnorm_mx(x, r, nw, 1e-6, oracle_mod.RULE_CEIL_DIV448)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(ac, as_, wc, ws, 0)))
    _check(y.float().cpu().numpy(), ref)
    assert np.array_equal(_bits(summed), rsum)
