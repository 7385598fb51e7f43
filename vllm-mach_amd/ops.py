"""Torch-facing operators over the gfx950 C ABI.

Every operator enqueues on the current HIP stream of its input's device,
allocates a fresh output per call, and is registered as a ``torch.library``
custom op whose fake implementation keeps the row count symbolic (the
contract of the reference's ``direct_register_custom_op`` ops, e.g.
src/vllm_mach/mxfp6/dense_mxfp8.py:99-111 and mxfp8/native_backend.py:208-220).
Scratch memory (split-K partials, routing counts) lives in per-(device, stream, kind)
workspaces that grow outside graph capture and raise inside it when a shape was not
warmed (mxfp8/native_backend.py:159-189).  A workspace handed to a call made during
graph capture is never freed: when a later shape outgrows it, the old buffer is kept
alive, because a captured graph still writes through its address on every replay.
``warmup`` (below) sizes every workspace to the largest shape of a model before
capture, as the reference's planning pass does (mxfp6/dense_mxfp8.py:177-220,
mxfp6/warmup.py:75-147).
"""
from __future__ import annotations

import contextlib
import ctypes
import threading
from typing import Optional

import torch

from . import _lib
from ._lib import call, ptr, query, stream_handle

E4M3, E2M3, E3M2 = 0, 2, 3
FLOOR_CARRY175, CEIL_DIV448, RP_UE8M0 = 0, 1, 2
FORMATS = {"e4m3": E4M3, "e2m3": E2M3, "e3m2": E3M2}

_ws_lock = threading.RLock()


class _Workspace:
    __slots__ = ("buf", "captured")

    def __init__(self, buf: torch.Tensor):
        self.buf = buf
        self.captured = False  # handed to a call during graph capture: a graph may hold its address


# (device index, stream handle, kind) -> the current workspace
_workspaces: dict[tuple[int, int, str], _Workspace] = {}
# superseded workspaces that a captured graph may still reference (kept until exit)
_retired: list[torch.Tensor] = []
# (device index, kind) -> planned bytes: the high-water mark of the shapes warmed so far
_planned: dict[tuple[int, str], int] = {}
_COUNTS: dict[str, int] = {}


def _count(key: str) -> None:
    _COUNTS[key] = _COUNTS.get(key, 0) + 1


def inspect() -> dict:
    """Call counters (eager/capture invocations, not graph replays), workspace sizes per
    (device, stream, kind), planned high-water marks, and the retired buffers kept for
    captured graphs."""
    with _ws_lock:
        return {"counts": dict(_COUNTS),
                "workspaces": {**{f"{d}:{s:#x}:{kind}": w.buf.numel() for (d, s, kind), w in _workspaces.items()},
                               **{f"{d}:{s:#x}:combine": 4 * w.buf.numel() for (d, s), w in _counters.items()}},
                "planned": {f"{d}:{kind}": n for (d, kind), n in _planned.items()},
                "retired_bytes": sum(t.numel() * t.element_size() for t in _retired)}


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def workspace(device: torch.device, nbytes: int, kind: str = "gemm") -> Optional[torch.Tensor]:
    """Per-(device, stream, kind) scratch of at least ``nbytes``.

    Outside capture a workspace that is too small is replaced by one of at least the
    planned size (``warmup``) and twice the old one; the old buffer is freed only if no
    captured graph can reference it.  During capture a workspace is never reallocated:
    a shape that needs more raises (warm it first)."""
    if nbytes <= 0:
        return None
    di = _device_index(device)
    key = (di, stream_handle(device), kind)
    capturing = torch.cuda.is_current_stream_capturing()
    with _ws_lock:
        _planned[(di, kind)] = max(_planned.get((di, kind), 0), nbytes)
        ws = _workspaces.get(key)
        if ws is None or ws.buf.numel() < nbytes:
            if capturing:
                _count("capture_cache_miss")
                raise RuntimeError(
                    f"mach_amd {kind} workspace for stream {key[1]:#x} holds "
                    f"{0 if ws is None else ws.buf.numel()} bytes but this shape needs {nbytes}; "
                    "run the shape once (warmup) before graph capture")
            size = max(nbytes, _planned[(di, kind)], 0 if ws is None else 2 * ws.buf.numel())
            if ws is not None and ws.captured:
                _retired.append(ws.buf)
            ws = _Workspace(torch.empty(size, dtype=torch.uint8, device=device))
            _workspaces[key] = ws
            _count("workspace_miss")
        if capturing:
            ws.captured = True
        return ws.buf


def reserve_workspaces(device: torch.device) -> None:
    """Give the current stream of ``device`` every planned workspace at its planned size
    (the capture-stream registration of ``warmup_mxfp6_sm120_stream``,
    src/vllm_mach/mxfp6/warmup.py:119-147); call outside capture."""
    di = _device_index(device)
    with _ws_lock:
        for (d, kind), n in list(_planned.items()):
            if d == di:
                if kind == "combine":
                    combine_counters(device, n // 4)
                else:
                    workspace(device, n, kind)


# Kernel-selection override for tuning runs and tests (None: the library's cost model).
# Set through ``tuning()``; read once per GEMM call, never from the environment.
_tuning: Optional[_lib.GemmOptions] = None

KERNEL_AUTO, KERNEL_STREAM, KERNEL_WIDE, KERNEL_GENERIC, KERNEL_STREAM_WIDE, KERNEL_CHUNK = -1, 0, 1, 2, 3, 4


@contextlib.contextmanager
def tuning(kernel: int = KERNEL_AUTO, splits: int = 0, tile_n: int = 0, tile_m: int = 0, hybrid: bool = False,
           waves: int = 0):
    """Force the GEMM kernel / wide tile / K split of every GEMM call inside the block
    (``mxl_gemm_options``; the reference's tactic and splits overrides,
    src/vllm_mach/mxfp8/native_backend.py:29).  Grouped GEMMs read ``kernel`` (their
    schedule) and ``tile_m``; ``waves`` (4 or 8) picks the wide MX kernel's workgroup size.
    For tuning runs and tests."""
    global _tuning
    old = _tuning
    _tuning = _lib.GemmOptions(0, kernel, splits, tile_n, tile_m, int(hybrid), waves)
    try:
        yield _tuning
    finally:
        _tuning = old


def wide_tuning(cfg: Optional[str] = None, tile_m: int = 0):
    """``tuning`` from a wide-tile spec "NT,S" or "NT,1,h" (hybrid) and an m-tile count."""
    if not cfg:
        return tuning(tile_m=tile_m)
    parts = cfg.split(",")
    return tuning(tile_n=int(parts[0]), splits=int(parts[1]), tile_m=tile_m,
                  hybrid=len(parts) > 2 and parts[2] == "h")


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def _check_cuda(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("mach_amd operators need tensors on a HIP device")


# -------------------------------------------------------------- quantizers

@torch.library.custom_op("mach_amd::quantize_mxfp8", mutates_args=())
def quantize_mxfp8(x: torch.Tensor, rule: int = FLOOR_CARRY175) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 [M, K] -> (E4M3 codes [M, K], E8M0 scales u8 [M, K/32]).

    Replaces ``torch.ops.mxfp6.quantize_mxfp8`` / ``quantize_mxfp8_logical``
    (src/vllm_mach/mxfp6/dense_mxfp8.py:40, mxfp6/moe_utils.py:172-202).
    """
    _check_cuda(x)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] % 32:
        raise ValueError("quantize_mxfp8 needs a 2-D bf16 tensor with K % 32 == 0")
    if x.stride(1) != 1:
        x = x.contiguous()
    M, K = x.shape
    codes = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    scales = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
    if M:
        call("mxl_quantize_mxfp8", ptr(x), M, K, x.stride(0), rule, ptr(codes), ptr(scales),
             stream_handle(x.device))
    _count("quantize_mxfp8")
    return codes, scales


@quantize_mxfp8.register_fake
def _(x, rule=FLOOR_CARRY175):
    return (x.new_empty(x.shape, dtype=torch.float8_e4m3fn),
            x.new_empty((x.shape[0], x.shape[1] // 32), dtype=torch.uint8))


@torch.library.custom_op("mach_amd::quantize_mxfp6", mutates_args=())
def quantize_mxfp6(x: torch.Tensor, fmt: int = E2M3) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 [N, K] -> (packed FP6 u8 [N, 3K/4], E8M0 u8 [N, K/32]), OCP MX v1.0 floor rule.

    Replaces the offline MXFP6 quantizer behind the reference's checkpoints and tests
    (``mxfp6.quantize_mxfp6``, tests/native_mxfp6/test_moe.py:179-184).
    """
    _check_cuda(x)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] % 32:
        raise ValueError("quantize_mxfp6 needs a 2-D bf16 tensor with K % 32 == 0")
    if x.stride(1) != 1:
        x = x.contiguous()
    M, K = x.shape
    packed = torch.empty((M, K * 3 // 4), dtype=torch.uint8, device=x.device)
    scales = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
    if M:
        call("mxl_quantize_mxfp6", ptr(x), M, K, x.stride(0), fmt, ptr(packed), ptr(scales), stream_handle(x.device))
    _count("quantize_mxfp6")
    return packed, scales


@quantize_mxfp6.register_fake
def _(x, fmt=E2M3):
    return (x.new_empty((x.shape[0], x.shape[1] * 3 // 4), dtype=torch.uint8),
            x.new_empty((x.shape[0], x.shape[1] // 32), dtype=torch.uint8))


@torch.library.custom_op("mach_amd::swiglu_mxfp8", mutates_args=())
def swiglu_mxfp8(gate_up: torch.Tensor, rule: int = CEIL_DIV448,
                 swizzled: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """SwiGLU -> MXFP8 producer, gate_up bf16 [M, 2K] -> (E4M3 [M, K], scales).

    Replaces ``_triton_quantize`` (src/vllm_mach/mxfp6/mxfp8_mlp.py:113-127);
    ``swizzled=True`` writes the reference's swizzled scale buffer
    (mxfp8_mlp.py:107-110,122), otherwise logical [M, K/32].
    """
    _check_cuda(gate_up)
    if gate_up.dtype != torch.bfloat16 or gate_up.ndim != 2 or gate_up.shape[1] % 64:
        raise ValueError("swiglu_mxfp8 needs bf16 [M, 2K] with K % 32 == 0")
    gate_up = gate_up.contiguous()
    M, K = gate_up.shape[0], gate_up.shape[1] // 2
    codes = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=gate_up.device)
    if swizzled:
        scales = torch.empty((query("mxl_swizzled_scale_bytes", M, K),), dtype=torch.uint8, device=gate_up.device)
    else:
        scales = torch.empty((M, K // 32), dtype=torch.uint8, device=gate_up.device)
    if M:
        call("mxl_swiglu_mxfp8", ptr(gate_up), M, K, rule, int(swizzled), ptr(codes), ptr(scales),
             stream_handle(gate_up.device))
    _count("swiglu_mxfp8")
    return codes, scales


@swiglu_mxfp8.register_fake
def _(gate_up, rule=CEIL_DIV448, swizzled=False):
    M, K = gate_up.shape[0], gate_up.shape[1] // 2
    codes = gate_up.new_empty((M, K), dtype=torch.float8_e4m3fn)
    if swizzled:
        rows = (M + 127) // 128 * 128
        return codes, gate_up.new_empty((rows * ((K // 32 + 3) // 4) * 4,), dtype=torch.uint8)
    return codes, gate_up.new_empty((M, K // 32), dtype=torch.uint8)


def _norm_args(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, what: str):
    _check_cuda(x, weight, *([residual] if residual is not None else []))
    if (x.dtype != torch.bfloat16 or x.ndim != 2 or weight.dtype != torch.bfloat16
            or weight.numel() != x.shape[1] or (residual is not None and (residual.shape != x.shape
                                                                          or residual.dtype != x.dtype))):
        raise ValueError(f"{what} needs bf16 x [M, N], residual like x (or None) and bf16 weight [N]")
    if x.shape[1] % 32 or not 32 <= x.shape[1] <= 16384:
        raise ValueError(f"{what} needs 32 <= N <= 16384 with N % 32 == 0 (N={x.shape[1]})")
    return x.contiguous(), residual.contiguous() if residual is not None else None, weight.contiguous()


@torch.library.custom_op("mach_amd::rmsnorm_mxfp8", mutates_args=())
def rmsnorm_mxfp8(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                  rule: int = CEIL_DIV448, swizzled: bool = True
                  ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Residual add + Gemma RMSNorm -> MXFP8 producer (the contract of ``quantize``,
    src/vllm_mach/mxfp6/mxfp8_norm_quant.py:42-55): returns (E4M3 [M, N], scales, summed
    bf16 [M, N]).  Scales are the reference's swizzled buffer by default, logical [M, N/32]
    with ``swizzled=False``.  Without a residual, summed is x itself.
    """
    x, residual, weight = _norm_args(x, residual, weight, "rmsnorm_mxfp8")
    M, N = x.shape
    codes = torch.empty((M, N), dtype=torch.float8_e4m3fn, device=x.device)
    if swizzled:
        scales = torch.empty((query("mxl_swizzled_scale_bytes", M, N),), dtype=torch.uint8, device=x.device)
    else:
        scales = torch.empty((M, N // 32), dtype=torch.uint8, device=x.device)
    summed = torch.empty_like(x) if residual is not None else x.clone()
    if M:
        call("mxl_rmsnorm_mxfp8", ptr(x), ptr(residual), ptr(weight), M, N, float(eps), rule, int(swizzled),
             ptr(codes), ptr(scales), ptr(summed) if residual is not None else None, stream_handle(x.device))
    _count("rmsnorm_mxfp8")
    return codes, scales, summed


@rmsnorm_mxfp8.register_fake
def _(x, residual, weight, eps, rule=CEIL_DIV448, swizzled=True):
    M, N = x.shape
    codes = x.new_empty((M, N), dtype=torch.float8_e4m3fn)
    if swizzled:
        rows = (M + 127) // 128 * 128
        scales = x.new_empty((rows * ((N // 32 + 3) // 4) * 4,), dtype=torch.uint8)
    else:
        scales = x.new_empty((M, N // 32), dtype=torch.uint8)
    return codes, scales, torch.empty_like(x)


@torch.library.custom_op("mach_amd::gemma_rmsnorm", mutates_args=())
def gemma_rmsnorm(x: torch.Tensor, residual: Optional[torch.Tensor], weight: torch.Tensor,
                  eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Residual add + Gemma RMSNorm with a bf16 output (the contract of ``mach_gemma_norm``,
    src/vllm_mach/mxfp6/gemma_norm.py:32-46): returns (y, summed); summed is empty [0]
    without a residual, as in the reference."""
    x, residual, weight = _norm_args(x, residual, weight, "gemma_rmsnorm")
    M, N = x.shape
    y = torch.empty_like(x)
    summed = torch.empty_like(x) if residual is not None else x.new_empty((0,))
    if M:
        call("mxl_gemma_rmsnorm", ptr(x), ptr(residual), ptr(weight), M, N, float(eps), ptr(y),
             ptr(summed) if residual is not None else None, stream_handle(x.device))
    _count("gemma_rmsnorm")
    return y, summed


@gemma_rmsnorm.register_fake
def _(x, residual, weight, eps):
    return torch.empty_like(x), (torch.empty_like(x) if residual is not None else x.new_empty((0,)))


@torch.library.custom_op("mach_amd::quantize_block_fp8", mutates_args=())
def quantize_block_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token group-128 FP8 quantization -> (E4M3 [M, K], fp32 [M, K/128] stride (1, M)).

    Replaces ``_quantize_kernel.quantize_out`` (src/vllm_mach/fp8/_quantize_kernel.py:20-25).
    """
    _check_cuda(x)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] % 128:
        raise ValueError("quantize_block_fp8 needs bf16 [M, K] with K % 128 == 0")
    x = x.contiguous()
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((K // 128, M), dtype=torch.float32, device=x.device).t()
    if M:
        call("mxl_quantize_block_fp8", ptr(x), M, K, ptr(q), ptr(s), stream_handle(x.device))
    _count("quantize_block_fp8")
    return q, s


@quantize_block_fp8.register_fake
def _(x):
    M, K = x.shape
    return (x.new_empty((M, K), dtype=torch.float8_e4m3fn),
            x.new_empty((K // 128, M), dtype=torch.float32).t())


@torch.library.custom_op("mach_amd::silu_and_mul_per_block_quant", mutates_args=("out", "scales"))
def silu_and_mul_per_block_quant(out: torch.Tensor, input: torch.Tensor, scales: torch.Tensor,
                                 is_scale_transposed: bool) -> None:
    """SiLU(gate)*up -> block-FP8, in place; the contract of ``mach_fp8_activation::run``
    (native/fp8_activation/activation.cu:62-104): input bf16 [rows, 2H], out E4M3 [rows, H],
    scales fp32 [rows, H/128] contiguous or with stride (1, rows)."""
    _check_cuda(out, input, scales)
    rows, H2 = input.shape
    H = H2 // 2
    if (input.dtype != torch.bfloat16 or out.dtype != torch.float8_e4m3fn or scales.dtype != torch.float32
            or tuple(out.shape) != (rows, H) or tuple(scales.shape) != (rows, H // 128) or H % 128
            or not input.is_contiguous() or not out.is_contiguous()):
        raise ValueError("silu_and_mul_per_block_quant: unexpected dtype/shape/layout")
    # the kernel writes scale (r, g) at g * rows + r (transposed) or r * H/128 + g
    if is_scale_transposed:
        if (rows > 1 and scales.stride() != (1, rows)) or (rows == 1 and H > 128 and scales.stride(1) != 1):
            raise ValueError("transposed scales need stride (1, rows)")
    elif not scales.is_contiguous():
        raise ValueError("scales must be contiguous")
    if rows:
        call("mxl_silu_mul_block_fp8", ptr(input), rows, H, int(is_scale_transposed), ptr(out), ptr(scales),
             stream_handle(input.device))
    _count("silu_and_mul_per_block_quant")


@silu_and_mul_per_block_quant.register_fake
def _(out, input, scales, is_scale_transposed):
    return None


# ------------------------------------------------------------ weight layout

def pack_weight(codes: torch.Tensor, scales: Optional[torch.Tensor], fmt: int) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Logical checkpoint layout -> MFMA-tiled layout (load time, replaces ``pack_scales``,
    src/vllm_mach/mxfp6/dense_mxfp8.py:150-151 and dense.py:185-188).

    codes: E4M3 [N, K] (fmt 0) or packed FP6 u8 [N, 3K/4]; scales: E8M0 u8 [N, K/32] or None.
    Batched [E, N, ...] inputs are packed per expert into one contiguous buffer.
    """
    _check_cuda(codes, scales)
    if codes.ndim == 3:
        parts = [pack_weight(codes[e], None if scales is None else scales[e], fmt) for e in range(codes.shape[0])]
        w = torch.stack([p[0] for p in parts])
        s = None if scales is None else torch.stack([p[1] for p in parts])
        return w, s
    c = _u8(codes).contiguous()
    N = c.shape[0]
    K = c.shape[1] if fmt == E4M3 else c.shape[1] * 4 // 3
    tiled = torch.empty(query("mxl_tiled_weight_bytes", N, K, fmt), dtype=torch.uint8, device=c.device)
    tiled_s = None
    if scales is not None:
        s = _u8(scales).contiguous()
        if tuple(s.shape) != (N, K // 32):
            raise ValueError(f"scales must be [N, K/32] = [{N}, {K // 32}], got {tuple(s.shape)}")
        tiled_s = torch.empty(query("mxl_tiled_scale_bytes", N, K), dtype=torch.uint8, device=c.device)
    call("mxl_pack_weight", ptr(c), ptr(s) if scales is not None else None, N, K, fmt, ptr(tiled), ptr(tiled_s),
         stream_handle(c.device))
    return tiled, tiled_s


# -------------------------------------------------------------------- GEMMs

def _gemm_ws(device, M, N, K, fmt=E4M3, block=False, opts=None):
    if opts is None:
        nbytes = query("mxl_gemm_workspace_bytes", M, N, K)
    else:
        nbytes = query("mxl_gemm_workspace_bytes_ex", M, N, K, fmt, int(block), _lib.options_ptr(opts))
    buf = workspace(device, nbytes)
    return (ptr(buf), nbytes) if buf is not None else (None, 0)


def _mx_gemm_call(a8, sa8, M, w, sw, n, k, w_fmt, bias, out, ldc, opts, sa_layout=0):
    """mxl_mx_gemm (defaults) or mxl_mx_gemm_ex (a scale layout or a tuning override)."""
    dev = a8.device
    if opts is None and sa_layout == 0:
        ws, wsb = _gemm_ws(dev, M, n, k)
        call("mxl_mx_gemm", ptr(a8), ptr(sa8), M, ptr(w), ptr(sw), n, k, w_fmt, ptr(bias), ptr(out), ldc,
             ws, wsb, stream_handle(dev))
        return
    o = _lib.GemmOptions(sa_layout) if opts is None else _lib.GemmOptions(
        sa_layout, opts.kernel, opts.splits, opts.tile_n, opts.tile_m, opts.hybrid, opts.waves)
    ws, wsb = _gemm_ws(dev, M, n, k, w_fmt, False, o)
    call("mxl_mx_gemm_ex", ptr(a8), ptr(sa8), M, ptr(w), ptr(sw), n, k, w_fmt, ptr(bias), ptr(out), ldc,
         ws, wsb, _lib.options_ptr(o), stream_handle(dev))


@torch.library.custom_op("mach_amd::mx_gemm", mutates_args=())
def mx_gemm(a: torch.Tensor, sa: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, n: int, k: int,
            w_fmt: int, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Block-scaled MX GEMM on pre-quantized MXFP8 activations: y = A * W^T, bf16 [M, N].

    Replaces ``torch.ops.mxfp8_sm120.gemm(a, b, sa, sb)`` (src/vllm_mach/mxfp6/dense_mxfp8.py:86)
    and ``mxfp6::gemm_w6a8_pdl`` (src/vllm_mach/mxfp6/ar_norm.py:144-147).  a: E4M3 [M, K] row-major,
    sa: E8M0 [M, K/32]; w / sw: tiled weight (``pack_weight``).
    """
    _check_cuda(a, sa, w, sw, bias)
    a8 = _u8(a)
    if a8.ndim != 2 or a8.shape[1] != k or a8.stride(1) != 1 or a8.stride(0) != k:
        a8 = a8.contiguous()
        if a8.shape[1] != k:
            raise ValueError(f"activation K={a8.shape[1]} does not match weight K={k}")
    M = a8.shape[0]
    sa8 = _u8(sa).contiguous()
    if tuple(sa8.shape) != (M, k // 32):
        raise ValueError(f"activation scales must be [M, K/32] = [{M}, {k // 32}]")
    out = torch.empty((M, n), dtype=torch.bfloat16, device=a.device)
    if M:
        _mx_gemm_call(a8, sa8, M, w, sw, n, k, w_fmt, bias, out, n, _tuning)
    _count("mx_gemm")
    return out


@mx_gemm.register_fake
def _(a, sa, w, sw, n, k, w_fmt, bias=None):
    return a.new_empty((a.shape[0], n), dtype=torch.bfloat16)


def swiglu_row_fusable(m: int, k: int, rule: int, w_fmt: int = E4M3) -> bool:
    """Shapes ``mxl_swiglu_mx_gemm`` runs in one launch (M <= 16 rows; rules ceil_div448 and
    rp_ue8m0; the weight-streaming GEMM's K range, see ``mxl_producer_gemm_supported``)."""
    return 1 <= m <= 16 and bool(query("mxl_producer_gemm_supported", 0, m, k, rule, w_fmt))


def quant_row_fusable(m: int, k: int, rule: int, w_fmt: int = E4M3) -> bool:
    """Shapes ``mxl_quant_mx_gemm`` runs in one launch (M <= 16 rows, every MXFP8 scale rule;
    the weight-streaming GEMM's K range, see ``mxl_producer_gemm_supported``)."""
    return 1 <= m <= 16 and bool(query("mxl_producer_gemm_supported", 1, m, k, rule, w_fmt))


def quant_rows_inreg(m: int, k: int, rule: int, w_fmt: int = E4M3) -> bool:
    """Shapes whose MXFP8 quantization ``mxl_quant_mx_gemm`` runs inside the GEMM's own
    wavefronts (one row; or up to 16 rows at K <= 6144), the one-launch scheme that measured
    faster than the quantizer and GEMM as two launches."""
    return 1 <= m <= 16 and bool(query("mxl_producer_gemm_supported", 3, m, k, rule, w_fmt))


def block_row_fusable(m: int, k: int) -> bool:
    """Shapes ``mxl_block_fp8_quant_gemm`` runs in one launch (M <= 16 rows)."""
    return 1 <= m <= 16 and bool(query("mxl_producer_gemm_supported", 2, m, k, 0, E4M3))


def block_row_inreg(m: int, k: int) -> bool:
    """Shapes whose block-FP8 quantization ``mxl_block_fp8_quant_gemm`` runs inside the
    GEMM's own wavefronts (one row), the one-launch scheme that measured faster than the
    quantizer and GEMM as two launches."""
    return m == 1 and bool(query("mxl_producer_gemm_supported", 4, m, k, 0, E4M3))


@torch.library.custom_op("mach_amd::quant_mx_gemm", mutates_args=())
def quant_mx_gemm(x: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, n: int, w_fmt: int,
                  rule: int = FLOOR_CARRY175, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """MXFP8 quantization -> MX GEMM of M <= 16 bf16 rows in one launch, bit-identical to
    ``quantize_mxfp8`` then ``mx_gemm`` (``mxfp8_sm120::gemm_from_float`` /
    ``mxfp6::gemm_from_float`` at decode sizes, src/vllm_mach/mxfp6/dense_mxfp8.py:89-96)."""
    _check_cuda(x, w, sw, bias)
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError("quant_mx_gemm needs bf16 [M, K]")
    x = x.contiguous()
    M, K = x.shape
    if not quant_row_fusable(M, K, rule, w_fmt):
        raise ValueError(f"quant_mx_gemm runs M <= 16 rows of the one-launch shapes "
                         f"(M={M}, K={K}, rule={rule}, w_fmt={w_fmt})")
    out = torch.empty((M, n), dtype=torch.bfloat16, device=x.device)
    call("mxl_quant_mx_gemm", ptr(x), M, K, rule, ptr(w), ptr(sw), n, w_fmt, ptr(bias), ptr(out), n,
         stream_handle(x.device))
    _count("quant_mx_gemm")
    return out


@quant_mx_gemm.register_fake
def _(x, w, sw, n, w_fmt, rule=FLOOR_CARRY175, bias=None):
    return x.new_empty((x.shape[0], n), dtype=torch.bfloat16)


@torch.library.custom_op("mach_amd::swiglu_mx_gemm", mutates_args=())
def swiglu_mx_gemm(gate_up: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, n: int, w_fmt: int,
                   rule: int = CEIL_DIV448, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """SwiGLU -> MXFP8 -> MX GEMM of M <= 16 rows in one launch, bit-identical to
    ``swiglu_mxfp8`` then ``mx_gemm`` (``mach_swiglu_mxfp8_down`` / ``mxfp6::gemm_from_swiglu``
    at decode sizes, src/vllm_mach/mxfp6/mxfp8_mlp.py:15-22, src/vllm_mach/mxfp6/fused_mlp.py:13-19)."""
    _check_cuda(gate_up, w, sw, bias)
    if gate_up.dtype != torch.bfloat16 or gate_up.ndim != 2 or gate_up.shape[1] % 64:
        raise ValueError("swiglu_mx_gemm needs bf16 [M, 2K]")
    gate_up = gate_up.contiguous()
    M, K = gate_up.shape[0], gate_up.shape[1] // 2
    if not swiglu_row_fusable(M, K, rule, w_fmt):
        raise ValueError(f"swiglu_mx_gemm runs M <= 16 rows of the one-launch shapes, rule 1 or 2 "
                         f"(M={M}, K={K}, rule={rule}, w_fmt={w_fmt})")
    out = torch.empty((M, n), dtype=torch.bfloat16, device=gate_up.device)
    call("mxl_swiglu_mx_gemm", ptr(gate_up), M, K, rule, ptr(w), ptr(sw), n, w_fmt, ptr(bias), ptr(out), n,
         stream_handle(gate_up.device))
    _count("swiglu_mx_gemm")
    return out


@swiglu_mx_gemm.register_fake
def _(gate_up, w, sw, n, w_fmt, rule=CEIL_DIV448, bias=None):
    return gate_up.new_empty((gate_up.shape[0], n), dtype=torch.bfloat16)


@torch.library.custom_op("mach_amd::block_fp8_quant_gemm", mutates_args=())
def block_fp8_quant_gemm(x: torch.Tensor, w: torch.Tensor, sb: torch.Tensor, n: int,
                         bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Block-FP8 activation quantization -> block-FP8 GEMM of M <= 16 bf16 rows in one launch,
    bit-identical to ``quantize_block_fp8`` then ``block_fp8_gemm`` (the per-token-group
    quantization + scaled GEMM pair, src/vllm_mach/fp8/linear.py:65-81,157-216)."""
    _check_cuda(x, w, sb, bias)
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise ValueError("block_fp8_quant_gemm needs bf16 [M, K]")
    x = x.contiguous()
    M, K = x.shape
    if not block_row_fusable(M, K):
        raise ValueError(f"block_fp8_quant_gemm runs M <= 16 rows of the one-launch shapes (M={M}, K={K})")
    out = torch.empty((M, n), dtype=torch.bfloat16, device=x.device)
    call("mxl_block_fp8_quant_gemm", ptr(x), M, K, ptr(w), ptr(sb), n, ptr(bias), ptr(out), n,
         stream_handle(x.device))
    _count("block_fp8_quant_gemm")
    return out


@block_fp8_quant_gemm.register_fake
def _(x, w, sb, n, bias=None):
    return x.new_empty((x.shape[0], n), dtype=torch.bfloat16)


@torch.library.custom_op("mach_amd::quantize_mxfp8_dual", mutates_args=())
def quantize_mxfp8_dual(x: torch.Tensor, rule: int = FLOOR_CARRY175
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Two-limb MXFP8 activations (the contract of the reference's dual ``quantize``,
    src/vllm_mach/mxfp8/dual.py:45-47): bf16 [M, K] -> (hi E4M3 [M, K], hi scales [M, K/32],
    residual E4M3 [M, K], residual scales [M, K/32]); residual = bf16(x - dequant(hi))."""
    _check_cuda(x)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] % 32:
        raise ValueError("quantize_mxfp8_dual needs bf16 [M, K] with K % 32 == 0")
    x = x.contiguous()
    M, K = x.shape
    hi = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    res = torch.empty_like(hi)
    s_hi = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
    s_res = torch.empty_like(s_hi)
    if M:
        call("mxl_quantize_mxfp8_dual", ptr(x), M, K, K, rule, ptr(hi), ptr(s_hi), ptr(res), ptr(s_res),
             stream_handle(x.device))
    _count("quantize_mxfp8_dual")
    return hi, s_hi, res, s_res


@quantize_mxfp8_dual.register_fake
def _(x, rule=FLOOR_CARRY175):
    M, K = x.shape
    codes = x.new_empty((M, K), dtype=torch.float8_e4m3fn)
    scales = x.new_empty((M, K // 32), dtype=torch.uint8)
    return codes, scales, torch.empty_like(codes), torch.empty_like(scales)


@torch.library.custom_op("mach_amd::mx_gemm_dual", mutates_args=())
def mx_gemm_dual(hi: torch.Tensor, s_hi: torch.Tensor, res: torch.Tensor, s_res: torch.Tensor, w: torch.Tensor,
                 sw: torch.Tensor, n: int, k: int, w_fmt: int, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Two-limb MX GEMM, M <= 64: y = bf16(hi . W^T + res . W^T), limbs accumulated in separate
    fp32 partials (the contract of the reference's dual ``gemm_out``,
    src/vllm_mach/mxfp8/dual.py:45-50; docs/mxfp8-champion.md:12)."""
    _check_cuda(hi, s_hi, res, s_res, w, sw, bias)
    h8, r8 = _u8(hi).contiguous(), _u8(res).contiguous()
    M = h8.shape[0]
    if h8.shape != r8.shape or h8.ndim != 2 or h8.shape[1] != k or M > 64:
        raise ValueError("mx_gemm_dual needs two [M, K] limbs with M <= 64 matching the weight's K")
    sh8, sr8 = _u8(s_hi).contiguous(), _u8(s_res).contiguous()
    if tuple(sh8.shape) != (M, k // 32) or tuple(sr8.shape) != (M, k // 32):
        raise ValueError(f"limb scales must be [M, K/32] = [{M}, {k // 32}]")
    out = torch.empty((M, n), dtype=torch.bfloat16, device=hi.device)
    if M:
        nbytes = 2 * M * n * 4
        buf = workspace(hi.device, nbytes)
        call("mxl_mx_gemm_dual", ptr(h8), ptr(sh8), ptr(r8), ptr(sr8), M, ptr(w), ptr(sw), n, k, w_fmt,
             ptr(bias), ptr(out), n, ptr(buf), nbytes, stream_handle(hi.device))
    _count("mx_gemm_dual")
    return out


@mx_gemm_dual.register_fake
def _(hi, s_hi, res, s_res, w, sw, n, k, w_fmt, bias=None):
    return hi.new_empty((hi.shape[0], n), dtype=torch.bfloat16)


def mx_gemm_from_float_dual(x: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, n: int, w_fmt: int,
                            rule: int = FLOOR_CARRY175, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Two-limb quantization then the two-limb GEMM (``_dual``, src/vllm_mach/mxfp8/dual.py:45-50)."""
    hi, s_hi, res, s_res = torch.ops.mach_amd.quantize_mxfp8_dual(x, rule)
    return torch.ops.mach_amd.mx_gemm_dual(hi, s_hi, res, s_res, w, sw, n, x.shape[1], w_fmt, bias)


def mx_gemm_from_float(x: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, n: int, w_fmt: int,
                       rule: int = FLOOR_CARRY175, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Quantize bf16 activations to MXFP8 and run the MX GEMM.

    Replaces ``mxfp8_sm120::gemm_from_float`` / ``mxfp6::gemm_from_float``
    (src/vllm_mach/mxfp6/dense_mxfp8.py:96, src/vllm_mach/mxfp6/dense.py:122-129).  Where
    the GEMM's own wavefronts can quantize (one row, or up to 16 rows at K <= 6144) it runs
    as one launch (``quant_mx_gemm``, the same bits); other shapes take the quantizer and
    the GEMM, which measured faster than the one-launch handoff ``quant_mx_gemm`` offers
    there.
    """
    if quant_rows_inreg(x.shape[0], x.shape[1], rule, w_fmt):
        return torch.ops.mach_amd.quant_mx_gemm(x, w, sw, n, w_fmt, rule, bias)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x, rule)
    return torch.ops.mach_amd.mx_gemm(a, sa, w, sw, n, x.shape[1], w_fmt, bias)


def swiglu_mx_down(gate_up: torch.Tensor, w: torch.Tensor, sw: torch.Tensor, n: int, w_fmt: int = E4M3,
                   rule: int = CEIL_DIV448) -> torch.Tensor:
    """SwiGLU -> MXFP8 producer then the down-projection GEMM (``mach_swiglu_mxfp8_down``,
    src/vllm_mach/mxfp6/mxfp8_mlp.py:15-22)."""
    if gate_up.shape[0] == 0:
        return gate_up.new_empty((0, n))
    if gate_up.shape[0] == 1 and swiglu_row_fusable(1, gate_up.shape[1] // 2, rule, w_fmt):
        return torch.ops.mach_amd.swiglu_mx_gemm(gate_up, w, sw, n, w_fmt, rule)
    a, sa = torch.ops.mach_amd.swiglu_mxfp8(gate_up, rule, False)
    return torch.ops.mach_amd.mx_gemm(a, sa, w, sw, n, gate_up.shape[1] // 2, w_fmt, None)


def norm_mx_gate_up(x: torch.Tensor, residual: Optional[torch.Tensor], norm_weight: torch.Tensor, eps: float,
                    w: torch.Tensor, sw: torch.Tensor, n: int, w_fmt: int = E4M3,
                    rule: int = CEIL_DIV448) -> tuple[torch.Tensor, torch.Tensor]:
    """Residual + Gemma RMSNorm -> MXFP8 producer then the gate_up GEMM; returns (gate_up,
    summed) like ``mach_norm_quant_mxfp8_gate_up`` (src/vllm_mach/mxfp6/mxfp8_norm_quant.py:58-72).
    The reference switches to an unquantized norm + float GEMM above 32 rows; here the
    MXFP8 producer serves every M."""
    a, sa, summed = torch.ops.mach_amd.rmsnorm_mxfp8(x, residual, norm_weight, eps, rule, False)
    if x.shape[0] == 0:
        return x.new_empty((0, n)), summed
    return torch.ops.mach_amd.mx_gemm(a, sa, w, sw, n, x.shape[1], w_fmt, None), summed


@torch.library.custom_op("mach_amd::block_fp8_gemm", mutates_args=())
def block_fp8_gemm(a: torch.Tensor, sa: torch.Tensor, w: torch.Tensor, sb: torch.Tensor, n: int, k: int,
                   bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Block-FP8 GEMM: y[m, n] = sum_g sa[m, g] sb[n/128, g] (A_g . W_g), bf16 out.

    Replaces ``vllm_mach_block_fp8::mm`` and the ``cutlass_scaled_mm`` route
    (src/vllm_mach/fp8/linear.py:65-81).  a E4M3 [M, K]; sa fp32 [M, K/128] with stride (1, M);
    w tiled (``pack_weight`` fmt 0, no scales); sb fp32 [ceil(N/128), K/128].
    """
    _check_cuda(a, sa, w, sb, bias)
    a8 = _u8(a).contiguous()
    M = a8.shape[0]
    if a8.shape[1] != k:
        raise ValueError("activation K does not match weight K")
    if tuple(sa.shape) != (M, k // 128) or sa.dtype != torch.float32:
        raise ValueError("sa must be fp32 [M, K/128]")
    # the kernels read sa[m, g] at g * M + m: column-major, which for one row means
    # consecutive groups (a row view of a wider column-major tensor is not)
    if (M > 1 and sa.stride() != (1, M)) or (M == 1 and k > 128 and sa.stride(1) != 1):
        sa = sa.t().contiguous().t()
    sb = sb.contiguous()
    out = torch.empty((M, n), dtype=torch.bfloat16, device=a.device)
    if M:
        opts = _tuning
        ws, wsb = _gemm_ws(a.device, M, n, k, E4M3, True, opts)
        if opts is None:
            call("mxl_block_fp8_gemm", ptr(a8), ptr(sa), M, ptr(w), ptr(sb), n, k, ptr(bias), ptr(out), n, ws, wsb,
                 stream_handle(a.device))
        else:
            call("mxl_block_fp8_gemm_ex", ptr(a8), ptr(sa), M, ptr(w), ptr(sb), n, k, ptr(bias), ptr(out), n, ws,
                 wsb, _lib.options_ptr(opts), stream_handle(a.device))
    _count("block_fp8_gemm")
    return out


@block_fp8_gemm.register_fake
def _(a, sa, w, sb, n, k, bias=None):
    return a.new_empty((a.shape[0], n), dtype=torch.bfloat16)


def block_fp8_from_float(x: torch.Tensor, w: torch.Tensor, sb: torch.Tensor, n: int,
                         bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Quantize bf16 activations to block-FP8 (fp32 scale per row per 128) and run the
    block-FP8 GEMM (the patched ``CutlassFp8BlockScaledMMKernel.apply_weights`` pair,
    src/vllm_mach/fp8/linear.py:157-216).  One row runs as one launch (every wavefront of
    the GEMM quantizes its own part of the row, the same bits); more rows take the two
    launches, which measured faster than the one-launch handoff ``block_fp8_quant_gemm``
    offers up to 16 rows."""
    if x.dtype == torch.bfloat16 and block_row_inreg(x.shape[0], x.shape[1]):
        return torch.ops.mach_amd.block_fp8_quant_gemm(x, w, sb, n, bias)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x)
    return torch.ops.mach_amd.block_fp8_gemm(q, s, w, sb, n, x.shape[1], bias)


# ---------------------------------------------------------------------- MoE

@torch.library.custom_op("mach_amd::moe_route", mutates_args=())
def moe_route(topk_ids: torch.Tensor, num_experts: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Stable token sort by expert -> (sorted_routes i32 [R], expert_offsets i64 [E+1], inverse i32 [R]).

    The routing contract of ``route_mxfp8_out`` (src/vllm_mach/mxfp6/moe_utils.py:205-255):
    expert_offsets, inverse_permutation; ids outside [0, E) are dropped (inverse -1).
    """
    _check_cuda(topk_ids)
    ids = topk_ids.to(torch.int32).contiguous()
    T, topk = ids.shape
    R = T * topk
    dev = ids.device
    sorted_routes = torch.empty(R, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int64, device=dev)
    inverse = torch.empty(R, dtype=torch.int32, device=dev)
    nbytes = query("mxl_moe_route_workspace_bytes", T, topk, num_experts)
    buf = workspace(dev, nbytes, "route")
    call("mxl_moe_route", ptr(ids), T, topk, num_experts, ptr(sorted_routes), ptr(offsets), ptr(inverse),
         ptr(buf), nbytes, stream_handle(dev))
    _count("moe_route")
    return sorted_routes, offsets, inverse


@moe_route.register_fake
def _(topk_ids, num_experts):
    R = topk_ids.shape[0] * topk_ids.shape[1]
    return (topk_ids.new_empty((R,), dtype=torch.int32),
            topk_ids.new_empty((num_experts + 1,), dtype=torch.int64),
            topk_ids.new_empty((R,), dtype=torch.int32))


@torch.library.custom_op("mach_amd::moe_router", mutates_args=())
def moe_router(router_logits: torch.Tensor, top_k: int, renormalize: bool = True
               ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Router logits [T, E] (fp32 or bf16) -> (topk_weights f32 [T, k], topk_ids i32 [T, k],
    sorted_routes i32 [T k], expert_offsets i64 [E+1], inverse i32 [T k]): softmax, top-k
    (ties to the lower expert), renormalization and the stable token sort of ``moe_route``,
    in one launch up to 1024 routes (vLLM's fused top-k softmax + the routing of
    ``route_mxfp8_out``, as qwen35_router_quant_out fuses them, src/vllm_mach/mxfp6/moe.py:142-152).
    """
    _check_cuda(router_logits)
    if router_logits.ndim != 2 or router_logits.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("moe_router needs fp32 or bf16 logits [T, E]")
    logits = router_logits.contiguous()
    T, E = logits.shape
    dev = logits.device
    weights = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    R = T * top_k
    sorted_routes = torch.empty(R, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int64, device=dev)
    inverse = torch.empty(R, dtype=torch.int32, device=dev)
    nbytes = query("mxl_moe_router_workspace_bytes", T, top_k, E)
    buf = workspace(dev, nbytes, "route")
    call("mxl_moe_router", ptr(logits), int(logits.dtype == torch.bfloat16), T, E, top_k, int(renormalize),
         ptr(weights), ptr(ids), ptr(sorted_routes), ptr(offsets), ptr(inverse), ptr(buf), nbytes,
         stream_handle(dev))
    _count("moe_router")
    return weights, ids, sorted_routes, offsets, inverse


@moe_router.register_fake
def _(router_logits, top_k, renormalize=True):
    T, E = router_logits.shape
    R = T * top_k
    return (router_logits.new_empty((T, top_k), dtype=torch.float32),
            router_logits.new_empty((T, top_k), dtype=torch.int32),
            router_logits.new_empty((R,), dtype=torch.int32),
            router_logits.new_empty((E + 1,), dtype=torch.int64),
            router_logits.new_empty((R,), dtype=torch.int32))


@torch.library.custom_op("mach_amd::grouped_gemm", mutates_args=())
def grouped_gemm(a: torch.Tensor, sa: torch.Tensor, row_index: Optional[torch.Tensor], row_div: int,
                 expert_offsets: torch.Tensor, routed_rows: int, w: torch.Tensor, sw: torch.Tensor,
                 n: int, k: int, w_fmt: int) -> torch.Tensor:
    """Grouped MX GEMM over experts (``grouped_gemm_w6a8_out``, src/vllm_mach/mxfp6/moe_utils.py:320-380).

    Output row p (sorted order) of expert e (expert_offsets[e] <= p < expert_offsets[e+1]) is
    A[row_index[p] // row_div] . W[e]^T, or A[p] . W[e]^T when row_index is None.
    Rows past expert_offsets[E] are left unwritten.
    """
    _check_cuda(a, sa, row_index, expert_offsets, w, sw)
    a8 = _u8(a).contiguous()
    sa8 = _u8(sa).contiguous()
    E = expert_offsets.shape[0] - 1
    out = torch.empty((routed_rows, n), dtype=torch.bfloat16, device=a.device)
    if routed_rows:
        opts = _tuning
        if opts is None:
            call("mxl_grouped_gemm", ptr(a8), ptr(sa8), a8.shape[0], ptr(row_index), row_div, ptr(expert_offsets),
                 E, routed_rows, ptr(w), ptr(sw), n, k, w_fmt, ptr(out), stream_handle(a.device))
        else:
            call("mxl_grouped_gemm_ex", ptr(a8), ptr(sa8), a8.shape[0], ptr(row_index), row_div,
                 ptr(expert_offsets), E, routed_rows, ptr(w), ptr(sw), n, k, w_fmt, ptr(out),
                 _lib.options_ptr(opts), stream_handle(a.device))
    _count("grouped_gemm")
    return out


@grouped_gemm.register_fake
def _(a, sa, row_index, row_div, expert_offsets, routed_rows, w, sw, n, k, w_fmt):
    return a.new_empty((routed_rows, n), dtype=torch.bfloat16)


def grouped_fused_supported(routed_rows: int, num_experts: int, k: int, w_fmt: int) -> bool:
    """Whether the grouped GEMMs with a fused activation producer run this shape."""
    return bool(query("mxl_grouped_fused_supported", routed_rows, num_experts, k, w_fmt))


@torch.library.custom_op("mach_amd::grouped_gemm_quant", mutates_args=())
def grouped_gemm_quant(x: torch.Tensor, row_index: Optional[torch.Tensor], row_div: int,
                       expert_offsets: torch.Tensor, routed_rows: int, w: torch.Tensor, sw: torch.Tensor,
                       n: int, k: int, w_fmt: int, rule: int = FLOOR_CARRY175) -> torch.Tensor:
    """MXFP8 quantization of the gathered bf16 rows fused into the grouped GEMM: bit-identical to
    ``quantize_mxfp8`` then ``grouped_gemm`` (the fused router-quant schedule's role,
    src/vllm_mach/mxfp6/moe.py:142-152)."""
    _check_cuda(x, row_index, expert_offsets, w, sw)
    if x.dtype != torch.bfloat16 or x.ndim != 2 or x.shape[1] != k or x.stride(1) != 1:
        raise ValueError("grouped_gemm_quant needs bf16 rows [T, K] with unit column stride")
    E = expert_offsets.shape[0] - 1
    out = torch.empty((routed_rows, n), dtype=torch.bfloat16, device=x.device)
    if routed_rows:
        call("mxl_grouped_gemm_quant", ptr(x), x.stride(0), ptr(row_index), row_div, ptr(expert_offsets), E,
             routed_rows, ptr(w), ptr(sw), n, k, w_fmt, rule, ptr(out), stream_handle(x.device))
    _count("grouped_gemm_quant")
    return out


@grouped_gemm_quant.register_fake
def _(x, row_index, row_div, expert_offsets, routed_rows, w, sw, n, k, w_fmt, rule=FLOOR_CARRY175):
    return x.new_empty((routed_rows, n), dtype=torch.bfloat16)


@torch.library.custom_op("mach_amd::grouped_gemm_swiglu", mutates_args=())
def grouped_gemm_swiglu(gate_up: torch.Tensor, expert_offsets: torch.Tensor, routed_rows: int, w: torch.Tensor,
                        sw: torch.Tensor, n: int, k: int, w_fmt: int, rule: int = CEIL_DIV448) -> torch.Tensor:
    """SwiGLU -> MXFP8 of the routed gate/up rows fused into the grouped GEMM: bit-identical to
    ``swiglu_mxfp8`` then ``grouped_gemm`` (``mxfp6_sm120_silu_grouped_gemm``,
    src/vllm_mach/mxfp6/moe_utils.py:383-442)."""
    _check_cuda(gate_up, expert_offsets, w, sw)
    if gate_up.dtype != torch.bfloat16 or gate_up.ndim != 2 or gate_up.shape[1] != 2 * k:
        raise ValueError("grouped_gemm_swiglu needs bf16 gate/up rows [R, 2K]")
    gate_up = gate_up.contiguous()
    E = expert_offsets.shape[0] - 1
    out = torch.empty((routed_rows, n), dtype=torch.bfloat16, device=gate_up.device)
    if routed_rows:
        call("mxl_grouped_gemm_swiglu", ptr(gate_up), ptr(expert_offsets), E, routed_rows, ptr(w), ptr(sw), n, k,
             w_fmt, rule, ptr(out), stream_handle(gate_up.device))
    _count("grouped_gemm_swiglu")
    return out


@grouped_gemm_swiglu.register_fake
def _(gate_up, expert_offsets, routed_rows, w, sw, n, k, w_fmt, rule=CEIL_DIV448):
    return gate_up.new_empty((routed_rows, n), dtype=torch.bfloat16)


@torch.library.custom_op("mach_amd::moe_reduce", mutates_args=("output",))
def moe_reduce(output: torch.Tensor, routed_output: torch.Tensor, topk_weights: torch.Tensor,
               inverse: torch.Tensor) -> None:
    """Weighted combine into ``output`` bf16 [T, H] (``moe_reduce_out``, src/vllm_mach/mxfp6/moe.py:697-702)."""
    _check_cuda(output, routed_output, topk_weights, inverse)
    T, H = output.shape
    topk = topk_weights.shape[1]
    if not output.is_contiguous():
        raise ValueError("moe_reduce needs a contiguous output")
    w = topk_weights.to(torch.float32).contiguous()
    y = routed_output.contiguous()
    inv = inverse.contiguous()
    call("mxl_moe_reduce", ptr(y), ptr(w), ptr(inv), T, topk, H, ptr(output), stream_handle(output.device))
    _count("moe_reduce")


@moe_reduce.register_fake
def _(output, routed_output, topk_weights, inverse):
    return None


# (device index, stream handle) -> zeroed int32 token counters of the combine-fused down
# projections (each launch leaves them zero); superseded buffers a graph may hold are kept
_counters: dict[tuple[int, int], _Workspace] = {}


def combine_counters(device: torch.device, tokens: int) -> torch.Tensor:
    """Per-(device, stream) int32 counters, zero, for ``tokens`` tokens: grown outside
    capture (zero-filled on the stream), never reallocated during capture (a miss raises,
    as a workspace miss does)."""
    di = _device_index(device)
    key = (di, stream_handle(device))
    capturing = torch.cuda.is_current_stream_capturing()
    with _ws_lock:
        _planned[(di, "combine")] = max(_planned.get((di, "combine"), 0), 4 * tokens)
        ws = _counters.get(key)
        if ws is None or ws.buf.numel() < tokens:
            if capturing:
                _count("capture_cache_miss")
                raise RuntimeError(f"mach_amd combine counters for stream {key[1]:#x} hold "
                                   f"{0 if ws is None else ws.buf.numel()} tokens but this call needs {tokens}; "
                                   "run the shape once (warmup) before graph capture")
            size = max(tokens, _planned[(di, "combine")] // 4, 0 if ws is None else 2 * ws.buf.numel())
            if ws is not None and ws.captured:
                _retired.append(ws.buf)
            ws = _Workspace(torch.zeros(size, dtype=torch.int32, device=device))
            _counters[key] = ws
            _count("workspace_miss")
        if capturing:
            ws.captured = True
        return ws.buf


def grouped_combine_supported(routed_rows: int, num_experts: int, n: int, k: int, w_fmt: int,
                              swiglu: bool, topk: int = 8) -> bool:
    """Whether a down projection with the weighted combine in its launch runs this shape
    (``swiglu``: with the SwiGLU producer fused as well): the small-batch schedule, at most
    16 routes per token."""
    return 1 <= topk <= 16 and bool(query("mxl_grouped_combine_supported", routed_rows, num_experts, n, k, w_fmt,
                                          2 if swiglu else 0))


def _combine_call(fn: str, output: torch.Tensor, routed_rows: int, n: int, sorted_routes: torch.Tensor,
                  inverse: torch.Tensor, topk_weights: torch.Tensor, *lead):
    T = output.shape[0]
    topk = topk_weights.shape[1]
    if output.dtype != torch.bfloat16 or tuple(output.shape) != (T, n) or not output.is_contiguous():
        raise ValueError(f"combine output must be contiguous bf16 [T, {n}]")
    if tuple(topk_weights.shape) != (T, topk) or inverse.numel() != T * topk:
        raise ValueError("topk_weights [T, topk] and inverse [T * topk] must match the output")
    dev = output.device
    y = torch.empty((routed_rows, n), dtype=torch.bfloat16, device=dev)
    w = topk_weights.to(torch.float32).contiguous()
    inv = inverse.contiguous()
    routes = sorted_routes.contiguous()
    cnt = combine_counters(dev, T)
    desc = _lib.MoeCombine(ptr(routes), ptr(inv), ptr(w), T, topk, ptr(output), ptr(cnt))
    call(fn, *lead, ptr(y), ctypes.byref(desc), stream_handle(dev))


@torch.library.custom_op("mach_amd::grouped_gemm_combine", mutates_args=("output",))
def grouped_gemm_combine(output: torch.Tensor, a: torch.Tensor, sa: torch.Tensor, row_index: Optional[torch.Tensor],
                         row_div: int, expert_offsets: torch.Tensor, routed_rows: int, w: torch.Tensor,
                         sw: torch.Tensor, n: int, k: int, w_fmt: int, sorted_routes: torch.Tensor,
                         inverse: torch.Tensor, topk_weights: torch.Tensor) -> None:
    """Grouped down projection (routed row p = A[row_index[p] // row_div] . W[e]^T, or A[p]
    without row_index) with the weighted combine in the same launch: ``output`` [T, n] =
    the bits of ``grouped_gemm`` then ``moe_reduce`` (grouped_gemm_w6a8_out + moe_reduce_out
    as one kernel, the role of the reference's array_gemm_w6a8_reduce_out,
    src/vllm_mach/mxfp6/moe.py:163-186)."""
    _check_cuda(output, a, sa, row_index, expert_offsets, w, sw, sorted_routes, inverse, topk_weights)
    a8 = _u8(a).contiguous()
    sa8 = _u8(sa).contiguous()
    E = expert_offsets.shape[0] - 1
    _combine_call("mxl_grouped_gemm_combine", output, routed_rows, n, sorted_routes, inverse, topk_weights,
                  ptr(a8), ptr(sa8), a8.shape[0], ptr(row_index), row_div, ptr(expert_offsets), E, routed_rows,
                  ptr(w), ptr(sw), n, k, w_fmt)
    _count("grouped_gemm_combine")


@grouped_gemm_combine.register_fake
def _(output, a, sa, row_index, row_div, expert_offsets, routed_rows, w, sw, n, k, w_fmt, sorted_routes, inverse,
      topk_weights):
    return None


@torch.library.custom_op("mach_amd::grouped_gemm_swiglu_combine", mutates_args=("output",))
def grouped_gemm_swiglu_combine(output: torch.Tensor, gate_up: torch.Tensor, expert_offsets: torch.Tensor,
                                routed_rows: int, w: torch.Tensor, sw: torch.Tensor, n: int, k: int, w_fmt: int,
                                rule: int, sorted_routes: torch.Tensor, inverse: torch.Tensor,
                                topk_weights: torch.Tensor) -> None:
    """SwiGLU -> MXFP8 of the routed gate/up rows, the grouped down projection and the
    weighted combine in one launch: ``output`` [T, n] = the bits of ``grouped_gemm_swiglu``
    then ``moe_reduce`` (the reference's qwen35_w2_splitk_reduce_out role,
    src/vllm_mach/mxfp6/moe.py:163-175)."""
    _check_cuda(output, gate_up, expert_offsets, w, sw, sorted_routes, inverse, topk_weights)
    if gate_up.dtype != torch.bfloat16 or gate_up.ndim != 2 or gate_up.shape[1] != 2 * k:
        raise ValueError("grouped_gemm_swiglu_combine needs bf16 gate/up rows [R, 2K]")
    gate_up = gate_up.contiguous()
    E = expert_offsets.shape[0] - 1
    _combine_call("mxl_grouped_gemm_swiglu_combine", output, routed_rows, n, sorted_routes, inverse, topk_weights,
                  ptr(gate_up), ptr(expert_offsets), E, routed_rows, ptr(w), ptr(sw), n, k, w_fmt, rule)
    _count("grouped_gemm_swiglu_combine")


@grouped_gemm_swiglu_combine.register_fake
def _(output, gate_up, expert_offsets, routed_rows, w, sw, n, k, w_fmt, rule, sorted_routes, inverse,
      topk_weights):
    return None
