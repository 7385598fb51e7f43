"""The reference's two-limb MXFP8 runtime module (``mxfp6.mxfp8_dual``) over this library.

src/vllm_mach/mxfp8/dual.py:40-50 calls ``quantize(x) -> (hi, s_hi, residual, s_res)``
and ``gemm_out(hi, weight, s_hi, scale.view(-1), residual, s_res, out)``; dual.py:109-111
calls ``load_library()``.  The limbs are this library's two-limb quantizer (high limb =
MXFP8(x), residual = MXFP8(bf16(x - dequant(high)))) with swizzled scales; ``gemm_out``
is ``torch.ops.mxfp8_sm120.dual_gemm_out`` (M <= 64).
"""
from __future__ import annotations

import torch

from . import mxfp6_api as _api

load_library = _api.load_library


def quantize(x: torch.Tensor):
    """bf16 [M, K] -> (hi E4M3 [M, K], swizzled s_hi, residual E4M3 [M, K], swizzled s_res)."""
    load_library()
    hi, s_hi, res, s_res = torch.ops.mach_amd.quantize_mxfp8_dual(x)
    return hi, torch.ops.mxfp6.pack_scales(s_hi), res, torch.ops.mxfp6.pack_scales(s_res)


def gemm_out(hi: torch.Tensor, weight: torch.Tensor, s_hi: torch.Tensor, s_weight: torch.Tensor,
             residual: torch.Tensor, s_res: torch.Tensor, out: torch.Tensor) -> None:
    """out[M, N] = bf16(hi . W^T + residual . W^T), summed in fp32 before the rounding."""
    load_library()
    torch.ops.mxfp8_sm120.dual_gemm_out(hi, weight, s_hi, s_weight, residual, s_res, out)
