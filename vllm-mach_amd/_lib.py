"""ctypes binding of the C ABI in ``include/mxlinear.h`` (``libmxlinear.so``).

The library is loaded lazily on first use, after ``import torch``, so that its
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch already
loaded and HIP stream handles are shared.  There is no fallback: a missing
library raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the library load; see module docstring)

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("MXLINEAR_LIBRARY_PATH", HERE / "libmxlinear.so"))

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/mxlinear.h
SIGNATURES = {
    "mxl_version": (_I, []),
    "mxl_last_error": (ctypes.c_char_p, []),
    "mxl_device_supported": (_I, [_I]),
    "mxl_quantize_mxfp8": (_I, [_P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "mxl_quantize_mxfp8_swizzled": (_I, [_P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "mxl_quantize_mxfp6": (_I, [_P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "mxl_swizzled_scale_bytes": (_I64, [_I64, _I64]),
    "mxl_swizzle_scales": (_I, [_P, _I64, _I64, _P, _P]),
    "mxl_swiglu_mxfp8": (_I, [_P, _I64, _I64, _I, _I, _P, _P, _P]),
    "mxl_quantize_mxfp8_dual": (_I, [_P, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P]),
    "mxl_mx_gemm_dual": (_I, [_P, _P, _P, _P, _I64, _P, _P, _I64, _I64, _I, _P, _P, _I64, _P, _I64, _P]),
    "mxl_mx_gemm_dual_ex": (_I, [_P, _P, _P, _P, _I64, _P, _P, _I64, _I64, _I, _P, _P, _I64, _P, _I64, _P, _P]),
    "mxl_rmsnorm_mxfp8": (_I, [_P, _P, _P, _I64, _I64, _F, _I, _I, _P, _P, _P, _P]),
    "mxl_gemma_rmsnorm": (_I, [_P, _P, _P, _I64, _I64, _F, _P, _P, _P]),
    "mxl_quantize_block_fp8": (_I, [_P, _I64, _I64, _P, _P, _P]),
    "mxl_silu_mul_block_fp8": (_I, [_P, _I64, _I64, _I, _P, _P, _P]),
    "mxl_tiled_weight_bytes": (_I64, [_I64, _I64, _I]),
    "mxl_tiled_scale_bytes": (_I64, [_I64, _I64]),
    "mxl_pack_weight": (_I, [_P, _P, _I64, _I64, _I, _P, _P, _P]),
    "mxl_pack_weight_ex": (_I, [_P, _P, _I, _I64, _I64, _I, _P, _P, _P]),
    "mxl_gemm_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "mxl_gemm_workspace_bytes_ex": (_I64, [_I64, _I64, _I64, _I, _I, _P]),
    "mxl_gemm_config_abi": (_I64, []),
    "mxl_set_gemm_config": (_I, [_I64, _I64, _I64, _I, _I, _P]),
    "mxl_clear_gemm_configs": (_I, []),
    "mxl_gemm_config_count": (_I64, []),
    "mxl_mx_gemm": (_I, [_P, _P, _I64, _P, _P, _I64, _I64, _I, _P, _P, _I64, _P, _I64, _P]),
    "mxl_noalloc_scratch_bytes": (_I64, []),
    "mxl_mx_gemm_noalloc": (_I, [_P, _P, _I64, _P, _P, _I64, _I64, _I, _P, _P, _I64, _P]),
    "mxl_mx_gemm_ex": (_I, [_P, _P, _I64, _P, _P, _I64, _I64, _I, _P, _P, _I64, _P, _I64, _P, _P]),
    "mxl_block_fp8_gemm_ex": (_I, [_P, _P, _I64, _P, _P, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _P]),
    "mxl_grouped_gemm_ex": (_I, [_P, _P, _I64, _P, _I, _P, _I64, _I64, _P, _P, _I64, _I64, _I, _P, _P, _P]),
    "mxl_swiglu_mx_gemm": (_I, [_P, _I64, _I64, _I, _P, _P, _I64, _I, _P, _P, _I64, _P]),
    "mxl_quant_mx_gemm": (_I, [_P, _I64, _I64, _I, _P, _P, _I64, _I, _P, _P, _I64, _P]),
    "mxl_swiglu_mx_gemm_ex": (_I, [_P, _I64, _I64, _I, _P, _P, _I64, _I, _P, _P, _I64, _P, _P]),
    "mxl_quant_mx_gemm_ex": (_I, [_P, _I64, _I64, _I, _P, _P, _I64, _I, _P, _P, _I64, _P, _P]),
    "mxl_block_fp8_gemm": (_I, [_P, _P, _I64, _P, _P, _I64, _I64, _P, _P, _I64, _P, _I64, _P]),
    "mxl_block_fp8_quant_gemm": (_I, [_P, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _P]),
    "mxl_block_fp8_quant_gemm_ex": (_I, [_P, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _P, _P]),
    "mxl_producer_gemm_supported": (_I, [_I, _I64, _I64, _I, _I]),
    "mxl_grouped_gemm": (_I, [_P, _P, _I64, _P, _I, _P, _I64, _I64, _P, _P, _I64, _I64, _I, _P, _P]),
    "mxl_grouped_fused_supported": (_I, [_I64, _I64, _I64, _I]),
    "mxl_grouped_gemm_quant": (_I, [_P, _I64, _P, _I, _P, _I64, _I64, _P, _P, _I64, _I64, _I, _I, _P, _P]),
    "mxl_grouped_gemm_swiglu": (_I, [_P, _P, _I64, _I64, _P, _P, _I64, _I64, _I, _I, _P, _P]),
    "mxl_grouped_combine_supported": (_I, [_I64, _I64, _I64, _I64, _I, _I]),
    "mxl_grouped_gemm_combine": (_I, [_P, _P, _I64, _P, _I, _P, _I64, _I64, _P, _P, _I64, _I64, _I, _P, _P, _P]),
    "mxl_grouped_gemm_swiglu_combine": (_I, [_P, _P, _I64, _I64, _P, _P, _I64, _I64, _I, _I, _P, _P, _P]),
    "mxl_moe_route_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "mxl_moe_route": (_I, [_P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "mxl_moe_reduce": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "mxl_moe_reduce_add": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P]),
    "mxl_moe_router_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "mxl_moe_router": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "mxl_gemm_plan_name": (_I, [_I64, _I64, _I64, _I, _I, _P, ctypes.c_char_p, _I64]),
    "mxl_grouped_plan_name": (_I, [_I64, _I64, _I64, _I, _I, _I, _P, ctypes.c_char_p, _I64]),
}

class GemmOptions(ctypes.Structure):
    """``mxl_gemm_options``: activation-scale layout, tuning overrides and output format of one
    GEMM call (out_dtype 0 bf16, 1 fp16; alpha the output scale)."""
    _fields_ = [("sa_layout", _I), ("kernel", _I), ("splits", _I), ("tile_n", _I), ("tile_m", _I),
                ("hybrid", _I), ("waves", _I), ("out_dtype", _I), ("alpha", _F)]

    def __init__(self, sa_layout=0, kernel=-1, splits=0, tile_n=0, tile_m=0, hybrid=0, waves=0, out_dtype=0,
                 alpha=1.0):
        super().__init__(sa_layout, kernel, splits, tile_n, tile_m, hybrid, waves, out_dtype, alpha)


class MoeCombine(ctypes.Structure):
    """``mxl_moe_combine``: the weighted combine a down projection runs in its own launch
    (routes, inverse, fp32 weights [T, topk], the bf16 [T, N] output, zeroed counters [T])."""
    _fields_ = [("sorted_routes", _P), ("inverse", _P), ("topk_weights", _P), ("T", _I64), ("topk", _I64),
                ("out", _P), ("counters", _P)]


def options_ptr(opts: "GemmOptions | None"):
    return None if opts is None else ctypes.byref(opts)


_lib = None
_lock = threading.Lock()


class MxlError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.is_file():
                    raise ImportError(
                        f"libmxlinear.so not found at {LIB_PATH}: build it with "
                        "`python vllm-mach_amd/build.py` (there is no CPU fallback)")
                L = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point; raise MxlError with its message on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().mxl_last_error().decode(errors="replace")
        raise MxlError(f"{name} failed ({rc}): {msg}")


def query(name: str, *args):
    return getattr(lib(), name)(*args)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def plan_name(fn: str, *args, options: "GemmOptions | None" = None) -> str:
    """The kernels ``mxl_gemm_plan_name`` / ``mxl_grouped_plan_name`` report for a call."""
    buf = ctypes.create_string_buffer(512)
    call(fn, *args, options_ptr(options), buf, len(buf))
    return buf.value.decode()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
