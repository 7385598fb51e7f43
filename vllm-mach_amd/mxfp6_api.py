"""The reference's native-library API over this library.

The reference binds its MX kernels through two kinds of native entry points:

* torch operators in a shared library that its loaders open with
  ``torch.ops.load_library`` and then check by schema (``mxfp8_sm120::*``,
  ``vllm_mach_block_fp8::mm``, ``mach_fp8_activation::run``, ``mxfp6::*``;
  src/vllm_mach/mxfp8/native_backend.py:76-125, src/vllm_mach/fp8/block_native.py:15-44,
  native/fp8_activation/activation.cu:98-104).  ``libmxlinear_torch.so`` registers
  those names and schemas over this library's C ABI; ``library_path()`` is the file a
  maintainer points ``MXFP8_LIBRARY_PATH`` / ``VLLM_MACH_BLOCK_FP8_LIBRARY`` at, and
  ``load_library()`` opens it.
* the Python API of the ``mxfp6`` package that the dense and MoE paths call
  (src/vllm_mach/mxfp6/moe_utils.py:15-44, 162-488; warmup.py:46-147;
  sm120_owner_prefill.py:50-63): ``MXFP8Tensor``, ``PackedMXFP6Tensor``,
  ``gemm_w6a8``, ``gemm_from_float``, ``warmup_w6a8``, ``autotune_w6a8``,
  ``quantize_mxfp8_logical``, ``quantize_mxfp8``, ``pack_scales``, ``to_mma_k64_weight``,
  ``route_mxfp8_out``, ``grouped_gemm_w6a8_out``, ``silu_and_mul_mxfp8_grouped``,
  ``moe_reduce_out`` and the workspace-planning calls, plus its runtime modules
  ``mxfp6.mxfp8`` (dense MXFP8, dense_mxfp8.py:45-220) and ``mxfp6.mxfp8_dual``
  (two-limb MXFP8, mxfp8/dual.py:40-50, 109-111) as the attributes ``mxfp8`` and
  ``mxfp8_dual``.  This module provides them with the same names, argument order and
  mutation contracts.  The Qwen3.5 TP2 schedules (``qwen35_*``,
  ``array_gemm_w6a8_reduce_out``, ``Qwen35GroupedWorkspace``) are multi-GPU and are
  not provided.

Layouts at this boundary are the reference's: weights stay in their checkpoint form
(E4M3 [N, K], packed FP6 [E, N, 3K/4]); weight scales are ``pack_scales`` output,
which here is the swizzled 128 x 4 layout (per expert for [E, R, K/32]).  The grouped
GEMMs read an MFMA-tiled copy of each expert weight tensor, made on first use outside
graph capture and kept while the weight tensor lives (invalidated when its version
changes).  ``route_mxfp8_out`` writes the permuted activation rows the reference's
grouped GEMM consumes; its "packed" scales are the routed rows' logical scales (the
buffer has the reference's size, rows + 127 per expert), and ``scale_offsets`` equals
``expert_offsets``, since these kernels need no per-expert padding.
"""
from __future__ import annotations

import threading
import weakref
from pathlib import Path
from typing import NamedTuple, Optional

import torch

from . import _lib, ops
from ._lib import call, ptr, query, stream_handle

HERE = Path(__file__).resolve().parent
TORCH_LIBRARY = HERE / "libmxlinear_torch.so"

# the reference's MXFP6 weights are E3M2 (Mxfp6Sm120LinearKernel, kMxfp6E3M2Static)
WEIGHT_FORMAT = ops.E3M2

_loaded = False
_lock = threading.Lock()


def library_path() -> str:
    """The torch operator library (``vllm_mach_block_fp8.library_path()`` /
    ``mxfp6.load_library()``'s artifact)."""
    return str(TORCH_LIBRARY)


def load_library() -> str:
    """Open the torch operator library once (registers the reference's op names)."""
    global _loaded
    with _lock:
        if not _loaded:
            if not TORCH_LIBRARY.is_file():
                raise ImportError(f"{TORCH_LIBRARY} not built: run `python vllm-mach_amd/build.py`")
            torch.ops.load_library(str(TORCH_LIBRARY))
            _loaded = True
    return library_path()


def is_available() -> bool:
    """A gfx950 device and a loadable library (fail closed)."""
    try:
        if not torch.cuda.is_available() or _lib.query("mxl_device_supported", torch.cuda.current_device()) != 1:
            return False
        load_library()
        return True
    except Exception:  # noqa: BLE001 - availability must fail closed
        return False


# ------------------------------------------------------------- quantizers

class MXFP8Tensor(NamedTuple):
    """An MXFP8 operand: E4M3 codes [rows, k] and its swizzled E8M0 scales
    (``mxfp6.MXFP8Tensor(values, scales, rows, k)``, sm120_owner_prefill.py:502,
    dense_mxfp8.py:214)."""
    values: torch.Tensor
    scales: torch.Tensor
    rows: int
    k: int


class PackedMXFP6Tensor(NamedTuple):
    """A packed MXFP6 (E3M2) weight: bytes [rows, 3k/4] and its swizzled E8M0 scales
    (``mxfp6.PackedMXFP6Tensor(values, scales, rows, k)``, warmup.py:55-60)."""
    values: torch.Tensor
    scales: torch.Tensor
    rows: int
    k: int


def quantize_mxfp8_logical(input: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 [M, K] -> (E4M3 [M, K], E8M0 u8 [M, K/32]) (moe_utils.py:172-202)."""
    return torch.ops.mach_amd.quantize_mxfp8(input, ops.FLOOR_CARRY175)


def quantize_mxfp8(input: torch.Tensor) -> MXFP8Tensor:
    """bf16 [M, K] -> codes and swizzled scales (``operand.values`` / ``.scales``,
    moe_utils.py:285-317)."""
    load_library()
    codes, scales = torch.ops.mxfp6.quantize_mxfp8(input)
    return MXFP8Tensor(codes, scales, int(input.shape[0]), int(input.shape[1]))


# ----------------------------------------------------------- dense W6A8

def _dtype(out_dtype) -> torch.dtype:
    """The GEMMs round their fp32 sums once to bf16 or fp16 (None: bf16)."""
    if out_dtype is None:
        return torch.bfloat16
    if out_dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"W6A8 GEMM output dtype must be bfloat16 or float16, got {out_dtype}")
    return out_dtype


def gemm_from_float(x: torch.Tensor, weight: PackedMXFP6Tensor, out_dtype=torch.bfloat16) -> torch.Tensor:
    """bf16 [M, K] quantized on the fly (floor_carry175) times a packed MXFP6 weight
    (tests/native_mxfp6/test_moe.py:232-241)."""
    load_library()
    return torch.ops.mxfp6.gemm_from_float(x, weight.values, weight.scales, int(weight.rows), 1.0, _dtype(out_dtype))


def gemm_w6a8(activation: MXFP8Tensor, weight: PackedMXFP6Tensor, out_dtype=torch.bfloat16) -> torch.Tensor:
    """A quantized MXFP8 activation (``quantize_mxfp8`` output) times a packed MXFP6
    weight (sm120_owner_prefill.py:61-63)."""
    load_library()
    codes = activation.values.view(torch.uint8) if activation.values.dtype != torch.uint8 else activation.values
    return torch.ops.mxfp6.gemm_w6a8_pdl(codes, weight.values, activation.scales, weight.scales, int(activation.rows),
                                         int(weight.rows), int(weight.k), 1.0, _dtype(out_dtype))


def warmup_w6a8(x: torch.Tensor, weight: PackedMXFP6Tensor, out_dtype=torch.bfloat16, iterations: int = 1) -> None:
    """Run the GEMM at x's shape (warmup.py:67): prepares the weight's tiled copy and
    grows this stream's workspace outside graph capture."""
    for _ in range(max(1, int(iterations))):
        gemm_from_float(x, weight, out_dtype=out_dtype)


def autotune_w6a8(x: torch.Tensor, weight: PackedMXFP6Tensor, out_dtype=torch.bfloat16, **_unused) -> None:
    """The reference tunes CUTLASS tactics per shape; here a cost model picks the kernel,
    so tuning is a warmup of the shape."""
    warmup_w6a8(x, weight, out_dtype=out_dtype)


def pack_scales(logical_scales: torch.Tensor) -> torch.Tensor:
    """Logical E8M0 [R, K/32] (or [E, R, K/32]) -> the swizzled layout (moe_utils.py:162-164)."""
    load_library()
    return torch.ops.mxfp6.pack_scales(logical_scales)


def to_mma_k64_weight(weight: torch.Tensor) -> torch.Tensor:
    """The reference's K = 64 TMA weight relayout (moe_utils.py:167-169).  The grouped
    GEMMs here tile every weight themselves, so the checkpoint layout is returned as is."""
    return weight


# ---------------------------------------------------------- tiled experts

_tiles: "weakref.WeakKeyDictionary[torch.Tensor, tuple]" = weakref.WeakKeyDictionary()


def _tiled_experts(weight: torch.Tensor, weight_scales: torch.Tensor, fmt: int):
    """MFMA-tiled copy of packed FP6 experts [E, N, 3K/4] with swizzled scales [E, S]."""
    if weight.ndim != 3 or weight.dtype != torch.uint8 or weight.shape[2] % 3:
        raise ValueError("expert weights must be packed FP6 bytes [E, N, 3K/4]")
    E, N, K = weight.shape[0], weight.shape[1], weight.shape[2] * 4 // 3
    stamp = (weight._version, weight_scales.data_ptr(), weight_scales._version, fmt)
    hit = _tiles.get(weight)
    if hit is not None and hit[0] == stamp:
        return hit[1], hit[2], N, K
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("expert weights were not prepared before graph capture; run the layer once first")
    per = query("mxl_swizzled_scale_bytes", N, K)
    ws = weight_scales.reshape(E, -1)
    if ws.shape[1] < per or ws.dtype not in (torch.uint8, torch.float8_e8m0fnu):
        raise ValueError(f"expert weight scales must be pack_scales output, {per} bytes per expert")
    w = weight.contiguous()
    ws = ws.contiguous().view(torch.uint8)
    wb, sb = query("mxl_tiled_weight_bytes", N, K, fmt), query("mxl_tiled_scale_bytes", N, K)
    tiled = torch.empty((E, wb), dtype=torch.uint8, device=w.device)
    tiled_s = torch.empty((E, sb), dtype=torch.uint8, device=w.device)
    st = stream_handle(w.device)
    for e in range(E):
        call("mxl_pack_weight_ex", ptr(w[e]), ptr(ws[e]), 1, N, K, fmt, ptr(tiled[e]), ptr(tiled_s[e]), st)
    _tiles[weight] = (stamp, tiled, tiled_s)
    return tiled, tiled_s, N, K


# ------------------------------------------------------------------- MoE

def route_mxfp8_out(activation: torch.Tensor, logical_scales: torch.Tensor, topk_ids: torch.Tensor,
                    expert_map: Optional[torch.Tensor], local_experts: int, permuted_activation: torch.Tensor):
    """Sort routes by expert and write the permuted activation rows (moe_utils.py:205-255).

    Returns (packed_scales, expert_offsets i64 [E+1], scale_offsets i64 [E+1],
    inverse_permutation i32 [T*topk]); routes whose (mapped) expert is outside
    [0, local_experts) are dropped (inverse -1).  ``permuted_activation`` [T*topk, K]
    receives row p = activation[route p's token] for the routed rows."""
    T, topk = topk_ids.shape
    K = activation.shape[1]
    ids = topk_ids if expert_map is None else expert_map[topk_ids.long()]
    sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_route(ids.to(torch.int32), local_experts)
    routes = T * topk
    tokens = torch.div(sorted_routes, topk, rounding_mode="floor").long()
    routed = int(routes)
    # rows past the routed count (dropped routes) keep whatever the buffer held
    valid = offsets[local_experts:local_experts + 1]
    keep = torch.arange(routed, device=tokens.device) < valid
    tokens = torch.where(keep, tokens, torch.zeros_like(tokens))
    pa = permuted_activation.view(torch.uint8).view(-1, K)[:routed]
    torch.index_select(activation.view(torch.uint8), 0, tokens, out=pa)
    packed = torch.empty(((routes + local_experts * 127) * (K // 32),), dtype=torch.uint8, device=activation.device)
    torch.index_select(logical_scales.view(torch.uint8), 0, tokens, out=packed[: routes * (K // 32)].view(routes, -1))
    return packed, offsets, offsets.clone(), inverse


def grouped_gemm_w6a8_out(output: torch.Tensor, activation: torch.Tensor, packed_scales: torch.Tensor,
                          weight: torch.Tensor, weight_scales: torch.Tensor, expert_offsets: torch.Tensor,
                          scale_offsets: torch.Tensor, *, fmt: int = WEIGHT_FORMAT) -> None:
    """output[p] = activation[p] . W[e]^T for the routed rows p of expert e
    (moe_utils.py:320-380); activation rows are the permuted rows of ``route_mxfp8_out``."""
    tiled, tiled_s, N, K = _tiled_experts(weight, weight_scales, fmt)
    E = expert_offsets.shape[0] - 1
    routes = activation.shape[0]
    if output.shape[1] != N or not output.is_contiguous() or output.dtype != torch.bfloat16:
        raise ValueError("output must be contiguous bf16 [routes, N]")
    a = activation.view(torch.uint8).contiguous()
    sa = packed_scales.view(torch.uint8)[: routes * (K // 32)]
    if routes:
        call("mxl_grouped_gemm", ptr(a), ptr(sa), routes, None, 1, ptr(expert_offsets), E, routes, ptr(tiled),
             ptr(tiled_s), N, K, fmt, ptr(output), stream_handle(output.device))


def silu_and_mul_mxfp8_grouped(gate_up: torch.Tensor, expert_offsets: torch.Tensor, scale_offsets: torch.Tensor):
    """SiLU(gate) * up -> MXFP8 over the routed rows (the reference test's arithmetic:
    SiLU rounded to bf16 before the product, ceil_div448 scales; moe_utils.py:383-442).
    Returns (E4M3 [routes, I], scales, scale_offsets)."""
    codes, scales = torch.ops.mach_amd.swiglu_mxfp8(gate_up, ops.CEIL_DIV448, False)
    return codes, scales, scale_offsets


def moe_reduce_out(output: torch.Tensor, routed_output: torch.Tensor, topk_weights: torch.Tensor,
                   inverse_permutation: torch.Tensor) -> None:
    """output[t] = bf16(sum_k w[t, k] y[inverse[t*topk + k]]) in fp32 (moe.py:697-702)."""
    torch.ops.mach_amd.moe_reduce(output, routed_output, topk_weights, inverse_permutation)


# ---------------------------------------------------- workspace planning

def begin_workspace_planning(device) -> None:
    """Start a planning pass (``warmup_mxfp8`` / ``warmup_mxfp6_sm120``): workspaces grow
    to every warmed shape's need and are never freed once a capture used them."""
    return None


def finalize_workspace_planning(device) -> None:
    """End a planning pass: give the current stream every planned workspace at its size."""
    ops.reserve_workspaces(torch.device(device) if not isinstance(device, torch.device) else device)


def workspace_stats(device) -> dict:
    """Planned and held workspace bytes (``mxfp6.workspace_stats``): ``lanes`` counts the
    (stream, kind) workspaces held."""
    info = ops.inspect()
    return {"lanes": len(info["workspaces"]), **info}


# the package's runtime submodules (``mxfp6.mxfp8``, ``mxfp6.mxfp8_dual``)
from . import mxfp8_api as mxfp8  # noqa: E402
from . import mxfp8_dual_api as mxfp8_dual  # noqa: E402
