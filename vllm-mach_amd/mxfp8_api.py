"""The reference's dense MXFP8 runtime module (``mxfp6.mxfp8``) over this library.

The reference's MXFP8 linear kernel imports it (src/vllm_mach/mxfp6/dense_mxfp8.py:45-46)
and requires ``load_library``, ``gemm_from_float``, ``begin_workspace_planning``,
``finalize_workspace_planning``, ``warmup`` and ``MXFP8Tensor`` (dense_mxfp8.py:120-125),
plus ``pack_scales`` for its weight scales (dense_mxfp8.py:151).  Weights are logical
E4M3 [N, K] with swizzled E8M0 scales; the GEMMs run through the torch operator
library's ``mxfp8_sm120`` ops.
"""
from __future__ import annotations

import torch

from . import mxfp6_api as _api

MXFP8Tensor = _api.MXFP8Tensor
load_library = _api.load_library
is_available = _api.is_available
pack_scales = _api.pack_scales
begin_workspace_planning = _api.begin_workspace_planning
finalize_workspace_planning = _api.finalize_workspace_planning
workspace_stats = _api.workspace_stats


def quantize(x: torch.Tensor) -> MXFP8Tensor:
    """bf16 [M, K] -> E4M3 codes with swizzled scales (floor_carry175)."""
    return _api.quantize_mxfp8(x)


def gemm_from_float(x: torch.Tensor, weight: MXFP8Tensor, out_dtype=torch.bfloat16) -> torch.Tensor:
    """bf16 [M, K] quantized on the fly times an MXFP8 weight (values E4M3 [N, K],
    swizzled scales)."""
    load_library()
    y = torch.ops.mxfp8_sm120.gemm_from_float(x, weight.values, weight.scales)
    return y if out_dtype in (None, torch.bfloat16) else y.to(out_dtype)


def gemm(activation: MXFP8Tensor, weight: MXFP8Tensor, out_dtype=torch.bfloat16) -> torch.Tensor:
    """Quantized activation times an MXFP8 weight (both with swizzled scales)."""
    load_library()
    y = torch.ops.mxfp8_sm120.gemm(activation.values, weight.values, activation.scales, weight.scales)
    return y if out_dtype in (None, torch.bfloat16) else y.to(out_dtype)


def warmup(x: torch.Tensor, weight: MXFP8Tensor, out_dtype=torch.bfloat16, iterations: int = 1) -> None:
    """Run the GEMM at x's shape (dense_mxfp8.py:214-217): prepares the weight's tiled
    copy and grows this stream's workspace outside graph capture."""
    for _ in range(max(1, int(iterations))):
        gemm_from_float(x, weight, out_dtype=out_dtype)
