"""Warmup and workspace planning before graph capture.

The reference plans its native workspaces in two passes (src/vllm_mach/mxfp6/dense_mxfp8.py:177-220
``warmup_mxfp8``; src/vllm_mach/mxfp6/warmup.py:75-147 ``warmup_mxfp6_sm120`` /
``warmup_mxfp6_sm120_stream``): first every distinct layer shape runs once at every token
count (graph sizes plus 64..2048 up to the largest, since intermediate sizes pick other
split-K layouts) to record the high-water mark of each workspace, then the graph-capture
stream is registered with workspaces of that size, so capture never allocates.

Here the same two passes run the layers' own ``apply`` paths: ``warmup(model, sizes)``
runs each distinct problem at each size (zeros in, no host sync per call) and leaves the
current stream's workspaces at the planned maxima; ``warmup(model, sizes, stream=True)``
gives the current (capture) stream workspaces of the planned sizes without running
anything.  Layers are found by what ``process_weights_after_loading`` left on them:
``mxl_kernel`` (dense kernels of ``linear``) and ``mxl_experts`` (``moe.Mxfp6MoEMethod``).
"""
from __future__ import annotations

from typing import Iterable, Union

import torch

from . import ops
from . import tactics as _tactics

# extra prefill sizes whose split-K layouts the graph sizes alone would miss
# (the reference's set, src/vllm_mach/mxfp6/dense_mxfp8.py:206-209)
PREFILL_SIZES = (64, 128, 256, 512, 1024, 2048)


def _modules(model: Union[torch.nn.Module, Iterable[torch.nn.Module]]):
    if isinstance(model, torch.nn.Module):
        yield from model.modules()
    else:
        for m in model:
            yield from (m.modules() if isinstance(m, torch.nn.Module) else (m,))


def collect_problems(model) -> tuple[dict, dict]:
    """Distinct dense problems {(kernel class, N, K, format): layer} and MoE problems
    {(E, H, I, format, topk): layer} among the prepared layers of ``model``."""
    dense: dict = {}
    moe: dict = {}
    for layer in _modules(model):
        kernel = getattr(layer, "mxl_kernel", None)
        if kernel is not None and hasattr(layer, "mxl_shape"):
            n, k = layer.mxl_shape
            key = (type(kernel).__name__, n, k, getattr(layer, "mxl_format", None),
                   tuple(sorted(getattr(kernel, "dual_m", ()))))
            dense.setdefault(key, layer)
        experts = getattr(layer, "mxl_experts", None)
        if experts is not None and experts.shapes is not None:
            E, H, I = experts.shapes
            moe.setdefault((E, H, I, experts.fmt, int(getattr(layer, "top_k", 8))), layer)
    return dense, moe


def _sizes(token_sizes: Iterable[int]) -> list[int]:
    sizes = {int(m) for m in token_sizes if int(m) > 0}
    if not sizes:
        return []
    top = max(sizes)
    return sorted(sizes | {m for m in PREFILL_SIZES if m <= top}, reverse=True)


def _device_of(layer) -> torch.device:
    for name in ("weight", "w13_weight"):
        t = getattr(layer, name, None)
        if isinstance(t, torch.Tensor):
            return t.device
    raise ValueError("prepared layer holds no weight tensor")


@torch.inference_mode()
def warmup(model, token_sizes: Iterable[int], *, stream: bool = False, tactics: str = "auto") -> dict:
    """Plan and reserve the workspaces of every prepared layer in ``model`` (a module or
    an iterable of modules) for the token counts ``token_sizes``.

    ``stream=False`` (before capture): register the packaged per-shape GEMM table's
    entries for the model's dense problems (``tactics.prepare``, mode ``tactics``: "auto",
    "on" or "off"; the reference's warmup registers its projection table first,
    src/vllm_mach/mxfp6/warmup.py:110-112), run each distinct dense problem at every size and
    each MoE problem at every token count, then give the current stream workspaces of
    the planned maxima.  ``stream=True`` (on the capture stream, after a planning pass):
    give the current stream the planned workspaces without running anything.  Returns
    the problems, sizes and resulting workspace table (``ops.inspect()``)."""
    dense, moe = collect_problems(model)
    sizes = _sizes(token_sizes)
    devices = {_device_of(layer) for layer in list(dense.values()) + list(moe.values())}
    registered = 0
    if not stream:
        if dense and _tactics.TABLE.is_file():
            registered = _tactics.prepare(dense.keys(), mode=tactics, device=_device_of(next(iter(dense.values()))))
        for (cls, n, k, fmt, dual), layer in dense.items():
            for m in sizes:
                x = torch.zeros((m, k), device=_device_of(layer), dtype=torch.bfloat16)
                layer.mxl_kernel.apply_weights(layer, x)
        for (E, H, I, fmt, topk), layer in moe.items():
            dev = _device_of(layer)
            experts = layer.mxl_experts
            for t in sizes:
                hidden = torch.zeros((t, H), device=dev, dtype=torch.bfloat16)
                # every expert receives rows: the routing's largest workspace and the
                # grouped kernels' widest schedules
                ids = (torch.arange(t * topk, device=dev, dtype=torch.int32) % E).view(t, topk)
                weights = torch.full((t, topk), 1.0 / topk, device=dev, dtype=torch.float32)
                out = torch.empty_like(hidden)
                experts.apply(out, hidden, layer.w13_weight, layer.w2_weight, weights, ids, "silu", E, None,
                              None, None, None, None, None, False)
    for dev in devices:
        ops.reserve_workspaces(dev)
        torch.cuda.synchronize(dev)
    return {"dense": sorted(dense), "moe": sorted(moe), "sizes": sizes, "workspaces": ops.inspect(),
            "tactics": registered}


def warmup_mxfp8(model, token_sizes, *, stream: bool = False) -> dict:
    """``warmup_mxfp8(model, token_sizes, stream=...)`` (src/vllm_mach/mxfp6/dense_mxfp8.py:177-220)."""
    return warmup(model, token_sizes, stream=stream)


def warmup_mxfp6_sm120(model, token_sizes, dtype=torch.bfloat16) -> dict:
    """The planning pass of ``warmup_mxfp6_sm120`` (src/vllm_mach/mxfp6/warmup.py:75-116);
    outputs are bf16 (``dtype`` is accepted for the signature)."""
    return warmup(model, token_sizes, stream=False)


def warmup_mxfp6_sm120_stream(model, token_sizes, dtype=torch.bfloat16) -> dict:
    """The capture-stream registration of ``warmup_mxfp6_sm120_stream``
    (src/vllm_mach/mxfp6/warmup.py:119-147)."""
    return warmup(model, token_sizes, stream=True)
