"""The champion SwiGLU -> MXFP8 producer (src/vllm_mach/mxfp8/swiglu_quant.py:23-70).

``quantize(x)`` keeps the reference's contract: x is the contiguous bf16 gate/up
output [m, 2k] of a supported width (2k in {12288, 18432}, else RuntimeError);
m == 0 or m > 128 returns None (the caller keeps its compiled operations); otherwise
the result is (E4M3 codes [m, k], E8M0 scales in the swizzled layout, flat uint8 of
ceil(m/128)*128 * ceil(k/128)*4 bytes).  Arithmetic: one bf16 rounding of
(g / (1 + exp(-g))) * up (no SiLU rounding, swiglu_quant.py:56-57) and the rp_ue8m0
scale rule (swiglu_quant.py:58-66), on the HIP producer (rule 2 of
``torch.ops.mach_amd.swiglu_mxfp8``).
"""
from collections import Counter

import torch

from . import ops

_COUNTS: Counter = Counter()
_WIDTHS = (12288, 18432)


def quantize(x: torch.Tensor):
    if (x.ndim != 2 or x.dtype != torch.bfloat16 or not x.is_cuda
            or not x.is_contiguous() or x.shape[1] not in _WIDTHS):
        raise RuntimeError("SwiGLU fusion requires a contiguous supported BF16 gate/up tensor")
    m = x.shape[0]
    _COUNTS[("capture" if torch.cuda.is_current_stream_capturing() else "eager", m)] += 1
    if m == 0 or m > 128:
        return None
    return torch.ops.mach_amd.swiglu_mxfp8(x, ops.RP_UE8M0, True)


def inspect() -> dict:
    """Call counts per (eager | capture, m), as the reference's receipts keep them."""
    return {"counts": {f"{mode}:{m}": n for (mode, m), n in sorted(_COUNTS.items())}}
