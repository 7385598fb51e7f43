"""MI355X-native (gfx950) quantized-linear hot path for vllm-mach.

Dynamic MXFP8 activation quantization, the SwiGLU -> MXFP8 producer, and the
block-scaled GEMMs for MXFP8, packed MXFP6 (W6A8) and block-FP8, dense and
MoE-grouped, as hand-written HIP kernels behind a C ABI (``include/mxlinear.h``,
``libmxlinear.so``) and vLLM's quantization-method surface (``linear``, ``moe``),
with loaders for the checkpoint formats that feed it (``checkpoint``).

Importing the package registers the ``torch.ops.mach_amd`` operators; it does
not touch the GPU or load the HIP library (that happens on first use).
"""
from . import ops  # noqa: F401  (registers torch.ops.mach_amd.*)
from . import swiglu_quant  # noqa: F401
from .linear import (  # noqa: F401
    BlockFp8LinearKernel,
    Mxfp6LinearKernel,
    Mxfp8LinearKernel,
    MxLinearLayerConfig,
    MxLinearMethod,
    is_mi355x_available,
    register_kernels,
    swiglu_mxfp8_down,
)
from .moe import Mxfp6Experts, Mxfp6MoEMethod, select_experts  # noqa: F401
from . import tactics  # noqa: F401  (the measured per-shape GEMM table: tactics.prepare)
from . import warmup  # noqa: F401  (the module: warmup.warmup, warmup.collect_problems)
from .warmup import warmup_mxfp6_sm120, warmup_mxfp6_sm120_stream, warmup_mxfp8  # noqa: F401
from .checkpoint import (  # noqa: F401
    SafetensorsCheckpoint,
    linear_quant_key,
    load_linear,
    load_moe,
    moe_quant_key,
    quant_config_of,
)

__version__ = "0.1.0"
