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
  mutation contracts.  The rest of the MoE API the reference checks for
  (``_MOE_REQUIRED_API``, moe_utils.py:28-44: ``qwen35_*``, ``array_gemm_w6a8_reduce_out``,
  ``Qwen35GroupedWorkspace``) are single-GPU schedules over one rank's experts; they are
  provided over the same kernels for any shape those take (the router, the grouped GEMMs
  with fused producers, the down projection with the combine in its launch).

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
from pathlib import Path
from typing import NamedTuple, Optional

import torch
from torch.utils.weak import WeakTensorKeyDictionary

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

# keyed by tensor identity (a WeakKeyDictionary would compare colliding keys with the
# tensors' elementwise ==); an entry goes when its weight tensor does
_tiles = WeakTensorKeyDictionary()


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


# ------------------------------------------- fused and grouped MoE schedules
#
# The reference's native schedules (src/vllm_mach/mxfp6/moe.py:126-313; names in
# moe_utils.py:28-44) are written for one TP2 shard of a Qwen3.5 layer with a shared
# expert appended to the routed ones (moe.py:398-426: w13/w2/scales gain expert E,
# combined_gate = [router gate; shared expert gate]).  Their kernels are in the absent
# wheel, so the arithmetic below is this library's definition, for any shape the grouped
# kernels take (the unsharded c5 layer included):
#   * logits = bf16(hidden . combined_gate^T) (fp32 accumulation); routed_logits are its
#     first E columns, shared_gate the last;
#   * top-k of softmax(routed_logits) renormalized (the router kernel, ties to the lower
#     expert), MXFP8 input codes under floor_carry175;
#   * with a shared expert, each token has a (topk + 1)-th route to expert E weighted
#     sigmoid(shared_gate) (binary32), combined last;
#   * routed activations SwiGLU -> MXFP8 under ceil_div448 (bf16 SiLU), as the layer's;
#   * the combine sums a token's routes in route order in fp32 and rounds once.


# The combine inside the down projection's launch (the reference's reduce-fused w2
# schedules); off by default: on MI355X the separate combine launch measured faster
# (c5 T = 128 layer 141.4 against 146.7 us).
FUSE_COMBINE = False


def _route_ext(topk_ids: torch.Tensor, topk_weights: Optional[torch.Tensor], routes: int, experts: int,
               shared_gate: Optional[torch.Tensor]):
    """Route table [T, k] with the shared expert's route appended when ``routes`` holds
    T * (topk + 1) rows; its weight sigmoid(shared_gate)."""
    T, topk = topk_ids.shape
    ids = topk_ids.to(torch.int32)
    wts = None if topk_weights is None else topk_weights.to(torch.float32)
    if routes == T * (topk + 1):
        ids = torch.cat([ids, torch.full((T, 1), experts - 1, dtype=torch.int32, device=ids.device)], 1)
        if wts is not None:
            if shared_gate is None:
                raise ValueError("a shared-expert route needs shared_gate")
            wts = torch.cat([wts, torch.sigmoid(shared_gate.float().reshape(T, 1))], 1)
    elif routes != T * topk:
        raise ValueError(f"{routes} routed rows for {T} tokens x {topk} routes")
    return ids.contiguous(), None if wts is None else wts.contiguous()


def qwen35_router_quant_out(quantized: torch.Tensor, input_scales: torch.Tensor, routed_logits: torch.Tensor,
                            topk_weights: torch.Tensor, topk_ids: torch.Tensor, shared_gate: torch.Tensor,
                            hidden_states: torch.Tensor, combined_gate: torch.Tensor, renormalize: bool = True) -> None:
    """Router GEMM, softmax top-k and MXFP8 input quantization (moe.py:142-152): writes
    every output argument.  ``combined_gate`` [E + 1, H] bf16 (the routed gate rows, then
    the shared expert's gate row)."""
    T, H = hidden_states.shape
    E = routed_logits.shape[1]
    if combined_gate.shape != (E + 1, H) or shared_gate.numel() != T:
        raise ValueError("combined_gate must be [E + 1, H] with shared_gate [T]")
    logits = torch.matmul(hidden_states, combined_gate.t())
    routed_logits.copy_(logits[:, :E])
    shared_gate.copy_(logits[:, E].reshape(shared_gate.shape))
    w, ids, _, _, _ = torch.ops.mach_amd.moe_router(routed_logits, topk_ids.shape[1], renormalize)
    topk_weights.copy_(w)
    topk_ids.copy_(ids)
    call("mxl_quantize_mxfp8", ptr(hidden_states), T, H, hidden_states.stride(0), ops.FLOOR_CARRY175,
         ptr(quantized), ptr(input_scales), stream_handle(hidden_states.device))


def qwen35_w1_splitk_silu_mxfp8_out(activation: torch.Tensor, activation_scales: torch.Tensor,
                                    w1_partial: torch.Tensor, quantized: torch.Tensor, input_scales: torch.Tensor,
                                    w1: torch.Tensor, w1_scales: torch.Tensor, topk_ids: torch.Tensor) -> None:
    """Grouped gate_up GEMM of every route, SwiGLU -> MXFP8 (moe.py:153-162): activation
    [routes, I] E4M3 and activation_scales [routes, I/32] in route order (token-major,
    the shared expert's route last).  ``w1_partial`` is the reference's split-K scratch,
    unused here."""
    tiled, tiled_s, N, K = _tiled_experts(w1, w1_scales, WEIGHT_FORMAT)
    experts = w1.shape[0]
    routes = activation.shape[0]
    ids, _ = _route_ext(topk_ids, None, routes, experts, None)
    sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_route(ids, experts)
    gate_up = torch.ops.mach_amd.grouped_gemm(quantized, input_scales, sorted_routes, ids.shape[1], offsets, routes,
                                              tiled, tiled_s, N, K, WEIGHT_FORMAT)
    codes, scales = torch.ops.mach_amd.swiglu_mxfp8(gate_up, ops.CEIL_DIV448, False)
    # route r's row is sorted row inverse[r] (no route is dropped: every id is an expert)
    torch.index_select(codes.view(torch.uint8), 0, inverse.long(), out=activation.view(torch.uint8))
    torch.index_select(scales.view(torch.uint8), 0, inverse.long(), out=activation_scales.view(torch.uint8))


def _w2_reduce(output, activation, activation_scales, w2, w2_scales, topk_ids, topk_weights, shared_gate):
    tiled, tiled_s, N, K = _tiled_experts(w2, w2_scales, WEIGHT_FORMAT)
    experts = w2.shape[0]
    routes = activation.shape[0]
    ids, wts = _route_ext(topk_ids, topk_weights, routes, experts, shared_gate)
    sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_route(ids, experts)
    a, sa = activation.view(torch.uint8), activation_scales.view(torch.uint8)
    if FUSE_COMBINE and ops.grouped_combine_supported(routes, experts, N, K, WEIGHT_FORMAT, False, ids.shape[1]) \
            and output.is_contiguous():
        # routed row p gathers activation row sorted_routes[p]; the combine runs in the launch
        torch.ops.mach_amd.grouped_gemm_combine(output, a, sa, sorted_routes, 1, offsets, routes, tiled, tiled_s, N, K,
                                                WEIGHT_FORMAT, sorted_routes, inverse, wts)
    else:
        y = torch.ops.mach_amd.grouped_gemm(a, sa, sorted_routes, 1, offsets, routes, tiled, tiled_s, N, K,
                                            WEIGHT_FORMAT)
        torch.ops.mach_amd.moe_reduce(output, y, wts, inverse)


def qwen35_w2_splitk_reduce_out(output: torch.Tensor, w2_partial: torch.Tensor, activation: torch.Tensor,
                                activation_scales: torch.Tensor, w2: torch.Tensor, w2_scales: torch.Tensor,
                                topk_ids: torch.Tensor, topk_weights: torch.Tensor, shared_gate: torch.Tensor) -> None:
    """Grouped down projection of the routed activations with the weighted combine
    (moe.py:163-175): output [T, H] bf16.  ``w2_partial`` (split-K scratch) is unused."""
    _w2_reduce(output, activation, activation_scales, w2, w2_scales, topk_ids, topk_weights, shared_gate)


def array_gemm_w6a8_reduce_out(output: torch.Tensor, activation: torch.Tensor, activation_scales: torch.Tensor,
                               w2: torch.Tensor, w2_scales: torch.Tensor, topk_ids: torch.Tensor,
                               topk_weights: torch.Tensor, shared_gate: torch.Tensor,
                               use_packed_vector_loads: bool = False) -> None:
    """The multi-token form of ``qwen35_w2_splitk_reduce_out`` (moe.py:176-186); the load
    width option is the reference kernel's and has no counterpart here."""
    _w2_reduce(output, activation, activation_scales, w2, w2_scales, topk_ids, topk_weights, shared_gate)


def qwen35_grouped_workspace_shapes(tokens: int, hidden: int = 2048, intermediate: int = 512, top_k: int = 8):
    """(workspace13, workspace2) shapes of the grouped schedule (moe.py:193-214): the
    routed gate/up rows [T k, 2I] and the routed down-projection rows [T k, H], bf16."""
    return (tokens * top_k, 2 * intermediate), (tokens * top_k, hidden)


class Qwen35GroupedWorkspace:
    """Buffers of the grouped schedule (moe.py:193-214): the layer output, the routed gate/up
    rows (workspace13) and routed output rows (workspace2), plus the routing of the last
    ``qwen35_grouped_gemm_out`` for ``qwen35_grouped_reduce_out``."""

    def __init__(self, output: torch.Tensor, workspace13: torch.Tensor, workspace2: torch.Tensor):
        self.output = output
        self.workspace13 = workspace13
        self.workspace2 = workspace2
        self.topk_weights: Optional[torch.Tensor] = None
        self.inverse: Optional[torch.Tensor] = None

    @classmethod
    def from_storage(cls, output: torch.Tensor, workspace13: torch.Tensor, workspace2: torch.Tensor):
        return cls(output, workspace13, workspace2)


def _grouped_gemms(workspace: Qwen35GroupedWorkspace, hidden_states, w1, w1_scales, w2, w2_scales,
                   weights, ids, sorted_routes, offsets, inverse, output: Optional[torch.Tensor]):
    """w13 (input quantization fused where the schedule takes it) into workspace13, then
    SwiGLU -> MXFP8 and w2 into workspace2, or with ``output`` the combine in w2's launch."""
    t1, s1, N1, K1 = _tiled_experts(w1, w1_scales, WEIGHT_FORMAT)
    t2, s2, N2, K2 = _tiled_experts(w2, w2_scales, WEIGHT_FORMAT)
    E = w1.shape[0]
    T, topk = ids.shape
    routes = T * topk
    gate_up = workspace.workspace13.reshape(-1)[: routes * N1].view(routes, N1)
    dev = hidden_states.device
    st = stream_handle(dev)
    if ops.grouped_fused_supported(routes, E, K1, WEIGHT_FORMAT) and hidden_states.stride(1) == 1:
        call("mxl_grouped_gemm_quant", ptr(hidden_states), hidden_states.stride(0), ptr(sorted_routes), topk,
             ptr(offsets), E, routes, ptr(t1), ptr(s1), N1, K1, WEIGHT_FORMAT, ops.FLOOR_CARRY175, ptr(gate_up), st)
    else:
        a, sa = torch.ops.mach_amd.quantize_mxfp8(hidden_states, ops.FLOOR_CARRY175)
        call("mxl_grouped_gemm", ptr(a), ptr(sa), T, ptr(sorted_routes), topk, ptr(offsets), E, routes, ptr(t1),
             ptr(s1), N1, K1, WEIGHT_FORMAT, ptr(gate_up), st)
    I = N1 // 2
    fused = ops.grouped_fused_supported(routes, E, I, WEIGHT_FORMAT)
    if output is not None and FUSE_COMBINE and ops.grouped_combine_supported(routes, E, N2, K2, WEIGHT_FORMAT,
                                                                              fused, topk):
        if fused:
            torch.ops.mach_amd.grouped_gemm_swiglu_combine(output, gate_up, offsets, routes, t2, s2, N2, K2,
                                                           WEIGHT_FORMAT, ops.CEIL_DIV448, sorted_routes, inverse,
                                                           weights)
        else:
            a2, sa2 = torch.ops.mach_amd.swiglu_mxfp8(gate_up, ops.CEIL_DIV448, False)
            torch.ops.mach_amd.grouped_gemm_combine(output, a2, sa2, None, 1, offsets, routes, t2, s2, N2, K2,
                                                    WEIGHT_FORMAT, sorted_routes, inverse, weights)
        return
    y = workspace.workspace2.reshape(-1)[: routes * N2].view(routes, N2)
    if fused:
        call("mxl_grouped_gemm_swiglu", ptr(gate_up), ptr(offsets), E, routes, ptr(t2), ptr(s2), N2, K2,
             WEIGHT_FORMAT, ops.CEIL_DIV448, ptr(y), st)
    else:
        a2, sa2 = torch.ops.mach_amd.swiglu_mxfp8(gate_up, ops.CEIL_DIV448, False)
        call("mxl_grouped_gemm", ptr(a2), ptr(sa2), routes, None, 1, ptr(offsets), E, routes, ptr(t2), ptr(s2), N2,
             K2, WEIGHT_FORMAT, ptr(y), st)
    if output is not None:
        torch.ops.mach_amd.moe_reduce(output, y, weights, inverse)


def qwen35_grouped_gemm_out(workspace: Qwen35GroupedWorkspace, hidden_states: torch.Tensor,
                            router_logits: torch.Tensor, w1: torch.Tensor, w1_scales: torch.Tensor, w2: torch.Tensor,
                            w2_scales: torch.Tensor, renormalize: bool = True) -> None:
    """The grouped schedule from router logits (moe.py:282-291): the router kernel (softmax,
    top-k, sort), w13 and w2 into the workspace; ``qwen35_grouped_reduce_out`` combines.
    The top-k is the workspace's routed rows per token."""
    T = hidden_states.shape[0]
    topk = workspace.workspace13.shape[0] // T if T else 1
    weights, ids, sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_router(router_logits, topk, renormalize)
    _grouped_gemms(workspace, hidden_states, w1, w1_scales, w2, w2_scales, weights, ids, sorted_routes, offsets,
                   inverse, None)
    workspace.topk_weights, workspace.inverse = weights, inverse


def qwen35_grouped_reduce_out(workspace: Qwen35GroupedWorkspace, output: torch.Tensor,
                              shared_output: Optional[torch.Tensor] = None) -> None:
    """Weighted combine of the workspace's routed rows into ``output`` (moe.py:296-302),
    with ``shared_output`` added to the fp32 sum before the one rounding."""
    if workspace.inverse is None:
        raise RuntimeError("qwen35_grouped_gemm_out must run before qwen35_grouped_reduce_out")
    T, H = output.shape
    topk = workspace.topk_weights.shape[1]
    y = workspace.workspace2.reshape(-1)[: T * topk * H].view(T * topk, H)
    if shared_output is None:
        torch.ops.mach_amd.moe_reduce(output, y, workspace.topk_weights, workspace.inverse)
        return
    if not output.is_contiguous() or shared_output.shape != output.shape:
        raise ValueError("output must be contiguous and shared_output of its shape")
    add = shared_output.to(torch.bfloat16).contiguous()
    call("mxl_moe_reduce_add", ptr(y), ptr(workspace.topk_weights), ptr(workspace.inverse), T, topk, H, ptr(add),
         ptr(output), stream_handle(output.device))


def qwen35_grouped_moe_out(workspace: Qwen35GroupedWorkspace, output: torch.Tensor, hidden_states: torch.Tensor,
                           w1: torch.Tensor, w1_scale: torch.Tensor, w2: torch.Tensor, w2_scale: torch.Tensor,
                           topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> None:
    """The routed layer from a given routing (moe_utils.py:47-74): sort, w13, w2 and the
    combine into ``output`` (the combine inside w2's launch where the schedule takes it)."""
    ids = topk_ids.to(torch.int32).contiguous()
    sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_route(ids, w1.shape[0])
    _grouped_gemms(workspace, hidden_states, w1, w1_scale, w2, w2_scale, topk_weights.to(torch.float32).contiguous(),
                   ids, sorted_routes, offsets, inverse, output)


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
