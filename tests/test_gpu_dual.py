"""GPU parity of the two-limb MXFP8 path (src/vllm_mach/mxfp8/dual.py:45-50): the
producer's four outputs are bit-exact against the oracle; the two-limb GEMM matches the
oracle's exact sum of both limbs' dequantize-then-matmul within the GEMM bar and is
closer to the bf16 dense product than the single-limb GEMM."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import _check, _weights

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def _x(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: K // 50]] *= 30
    return x.bfloat16()


@pytest.mark.parametrize("M,K,rule", [(1, 32, 0), (32, 2560, 0), (64, 2560, 1), (7, 5120, 0)])
def test_quantize_mxfp8_dual_bit_exact(pkg, oracle_mod, dev, M, K, rule):
    x = _x(M, K, 5 + M)
    got = torch.ops.mach_amd.quantize_mxfp8_dual(x.to(dev), rule)
    ref = oracle_mod.quant_mxfp8_dual(x, rule)
    for g, r in zip(got, ref):
        assert np.array_equal(_u8(g), r)


@pytest.mark.parametrize("M,N,K,fmt", [(32, 2048, 2560, 0), (64, 1024, 2560, 0), (5, 512, 1024, 2), (1, 256, 512, 0)])
def test_mx_gemm_dual(pkg, oracle_mod, dev, M, N, K, fmt):
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 31 + N)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _x(M, K, 9 + M)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(4)) * 0.5).bfloat16()
    y = ops.mx_gemm_from_float_dual(x.to(dev), tiled, tiled_s, N, fmt, 0, b.to(dev))
    hi, s_hi, res, s_res = oracle_mod.quant_mxfp8_dual(x, 0)
    ref = oracle_mod.mx_gemm_ref(hi, s_hi, wc, ws, fmt) + oracle_mod.mx_gemm_ref(res, s_res, wc, ws, fmt)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref))
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref + b.float().numpy()[None, :]))
    _check(y.float().cpu().numpy(), ref)
    # closer to the bf16 dense product than one limb
    dense = x.float().numpy() @ oracle_mod.dequant_mx(wc, ws, fmt).T + b.float().numpy()[None, :]
    one = ops.mx_gemm_from_float(x.to(dev), tiled, tiled_s, N, fmt, 0, b.to(dev)).float().cpu().numpy()
    e1 = np.linalg.norm(one - dense) / np.linalg.norm(dense)
    e2 = np.linalg.norm(y.float().cpu().numpy() - dense) / np.linalg.norm(dense)
    assert e2 < e1 / 2


def test_linear_kernel_dual_rows(pkg, oracle_mod, dev):
    """Mxfp8LinearKernel(dual_m=(32,)) serves M = 32 with two limbs, other M with one."""
    N, K = 512, 1024
    wc, ws, stored = _weights(oracle_mod, N, K, 0, 0.02, 3)
    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(torch.from_numpy(stored).view(torch.float8_e4m3fn).to(dev), requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(torch.from_numpy(ws).to(dev), requires_grad=False)
    kern = pkg.Mxfp8LinearKernel(dual_m=(32,))
    kern.process_weights_after_loading(layer)
    x32, x16 = _x(32, K, 1).to(dev), _x(16, K, 2).to(dev)
    assert torch.equal(kern.apply_weights(layer, x32),
                       pkg.ops.mx_gemm_from_float_dual(x32, layer.weight, layer.weight_scale, N, 0))
    assert torch.equal(kern.apply_weights(layer, x16),
                       pkg.ops.mx_gemm_from_float(x16, layer.weight, layer.weight_scale, N, 0))
