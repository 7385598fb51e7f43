"""Pins of the oracle's two-limb MXFP8 quantizer (the contract of
src/vllm_mach/mxfp8/dual.py:45-50 and docs/mxfp8-champion.md:12; the quantizer itself
lives in the absent mxfp6 wheel, so its rule is this build's definition and parity with
the reference is unpinned):

* the high limb is the single-limb quantizer's output, bit for bit (pinned by the stored
  KAT of quantize_block through test_oracle_quant);
* the residual limb is the single-limb quantizer applied to bf16(x - dequant(hi)), with
  dequant evaluated by torch's float8 decode and exact powers of two;
* the two limbs reconstruct x far more closely than the high limb alone.
"""
import numpy as np
import torch

import oracle


def _x(R, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(R, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: K // 50]] *= 30
    return x.bfloat16()


def test_high_limb_is_single_quantizer():
    x = _x(6, 1024, 1)
    for rule in (0, 1):
        hi, s_hi, _, _ = oracle.quant_mxfp8_dual(x, rule)
        c, s = oracle.quant_mxfp8(x, rule)
        assert np.array_equal(hi, c) and np.array_equal(s_hi, s)


def test_residual_limb_quantizes_bf16_remainder():
    x = _x(5, 512, 2)
    for rule in (0, 1):
        hi, s_hi, res, s_res = oracle.quant_mxfp8_dual(x, rule)
        deq = torch.from_numpy(hi).view(torch.float8_e4m3fn).float().view(5, 16, 32)
        deq = deq * torch.exp2(torch.from_numpy(s_hi.astype(np.float32)) - 127)[..., None]
        r = (x.float() - deq.view(5, 512)).bfloat16()
        c, s = oracle.quant_mxfp8(r, rule)
        assert np.array_equal(res, c) and np.array_equal(s_res, s)


def test_two_limbs_reconstruct_closer():
    x = _x(8, 2048, 3)
    hi, s_hi, res, s_res = oracle.quant_mxfp8_dual(x, 0)
    xf = x.float().numpy()
    one = oracle.dequant_mx(hi, s_hi, 0)
    two = one + oracle.dequant_mx(res, s_res, 0)
    e1 = np.linalg.norm(one - xf) / np.linalg.norm(xf)
    e2 = np.linalg.norm(two - xf) / np.linalg.norm(xf)
    assert e1 > 0.01 and e2 < e1 / 16
