"""MXFP6 (W6A8) routed-expert MoE on MI355X.

``Mxfp6Experts.apply`` keeps the signature and mutation contract of the
reference's ``Mxfp6Sm120Experts.apply`` (src/vllm_mach/mxfp6/moe.py:574-702):
quantize hidden states to MXFP8 -> stable token sort by expert -> grouped
W6A8 GEMM (w13) -> SwiGLU (bf16 SiLU) + MXFP8 -> grouped W6A8 GEMM (w2) ->
fp32 weighted combine into ``output``.  The grouped GEMMs gather activation
rows through the sorted route list, so no permuted copy of the activations is
written, and experts that receive no rows read no weights.  Where the grouped
weight-streaming schedules run (below ~96 routed rows per expert), they produce
their own MXFP8 operands -- the quantization inside w13, the SwiGLU inside w2 --
so a small-batch layer from router logits is four launches (router + sort, w13, w2,
combine).  The down projection can also run the weighted combine itself (each token's
row summed by the workgroup that stores its last routed row; ``fuse_combine``), which
makes it three launches with the same bits but measured slower on MI355X.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops

SILU = "silu"


def select_experts(router_logits: torch.Tensor, top_k: int, renormalize: bool = True):
    """softmax -> top-k -> optional renormalization (fp32 weights [T, k], int32 ids [T, k]),
    vLLM's ``select_experts`` with softmax scoring, in one router launch (``ops.moe_router``;
    ties go to the lower expert, as vLLM's top-k softmax kernel breaks them)."""
    weights, ids, _, _, _ = torch.ops.mach_amd.moe_router(router_logits, top_k, renormalize)
    return weights, ids


class Mxfp6Experts:
    """Routed experts over packed MXFP6 weights.

    Checkpoint layout (Quark OCP-MX): w13 u8 [E, 2I, 3H/4] + E8M0 [E, 2I, H/32] (gate rows
    [0, I), up rows [I, 2I)); w2 u8 [E, H, 3I/4] + E8M0 [E, H, I/32].  The weight format
    defaults to E3M2, the reference's (``Mxfp6Sm120Experts``); E2M3 is selected explicitly.
    """

    def __init__(self, fmt: int = ops.E3M2, act_rule: int = ops.FLOOR_CARRY175,
                 mid_rule: int = ops.CEIL_DIV448):
        if fmt not in (ops.E2M3, ops.E3M2):
            raise ValueError("MXFP6 MoE weights are E2M3 or E3M2")
        self.fmt = fmt
        self.act_rule = act_rule
        self.mid_rule = mid_rule
        self.fuse = True  # fused producers where the grouped schedule admits them (False: separate launches)
        # the weighted combine inside the down projection's launch (three launches from router
        # logits at small batch; the same bits).  Off by default: measured at c5 T = 128 the
        # layer takes 146.7 us with it against 141.4 us with the combine as its own launch --
        # each unit's end waits on its device-coherent stores, the token counter and the
        # routed rows' reads from beyond its XCD (w2 46.7 -> 58.4 us), more than a launch costs.
        self.fuse_combine = False
        self.w1_scale: Optional[torch.Tensor] = None
        self.w2_scale: Optional[torch.Tensor] = None
        self.shapes: Optional[tuple[int, int, int]] = None  # (E, H, I)

    def process_weights_after_loading(self, w13: torch.Tensor, w13_scale: torch.Tensor,
                                      w2: torch.Tensor, w2_scale: torch.Tensor):
        """Pack per-expert weights to the MFMA-tiled layout; returns (w1, w2) for ``apply``."""
        E, two_i, packed_h = w13.shape
        H = packed_h * 4 // 3
        I = two_i // 2
        if tuple(w2.shape) != (E, H, I * 3 // 4):
            raise ValueError("MXFP6 MoE weight shapes are inconsistent")
        if H % 128 or I % 128:
            raise ValueError("MXFP6 MoE needs hidden and intermediate sizes divisible by 128")
        w1_t, s1_t = ops.pack_weight(w13, w13_scale, self.fmt)
        w2_t, s2_t = ops.pack_weight(w2, w2_scale, self.fmt)
        self.w1_scale, self.w2_scale = s1_t, s2_t
        self.shapes = (E, H, I)
        return w1_t, w2_t

    def workspace_shapes(self, M: int, N: int, K: int, topk: int, global_num_experts: int,
                         local_num_experts: int, expert_tokens_meta=None, activation: str = SILU):
        """(workspace13, workspace2, output) shapes, as mxfp6/moe.py:543-572 computes them."""
        return (M * topk, max(N, K)), (M * topk, max(N // 2, K)), (M, K)

    def apply(self, output: torch.Tensor, hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
              topk_weights: torch.Tensor, topk_ids: torch.Tensor, activation: str, global_num_experts: int,
              expert_map: Optional[torch.Tensor], a1q_scale, a2_scale, workspace13, workspace2,
              expert_tokens_meta, apply_router_weight_on_input: bool) -> None:
        if apply_router_weight_on_input:
            raise ValueError("MXFP6 MoE requires router weights on output")
        if expert_tokens_meta is not None:
            raise ValueError("MXFP6 MoE requires standard routed activations")
        if activation != SILU:
            raise ValueError("MXFP6 MoE currently supports only SiLU")
        if self.shapes is None:
            raise RuntimeError("process_weights_after_loading must run before apply")
        E, H, I = self.shapes
        T, hidden = hidden_states.shape
        if hidden != H:
            raise ValueError("w1 packed K does not match the activation")
        if expert_map is None and global_num_experts != E:
            raise ValueError("global and local expert counts require an expert_map")
        ids = topk_ids if expert_map is None else expert_map[topk_ids.long()]
        topk = ids.shape[1]
        if T == 0:
            return
        sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_route(ids, E)
        self._experts(output, hidden_states, w1, w2, topk_weights, topk, sorted_routes, offsets, inverse)

    def apply_router(self, output: torch.Tensor, hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                     router_logits: torch.Tensor, top_k: int, renormalize: bool = True) -> None:
        """The layer from router logits [T, E]: one router launch (softmax, top-k,
        renormalization and the token sort, ``ops.moe_router``) feeds the grouped GEMMs
        directly, the reference's router-fused schedules (src/vllm_mach/mxfp6/moe.py:126-190,
        219-300: qwen35_router_quant_out routes before the expert GEMMs).  Writes ``output``;
        the same bits as ``select_experts`` then ``apply``."""
        if self.shapes is None:
            raise RuntimeError("process_weights_after_loading must run before apply")
        E, H, _ = self.shapes
        T, hidden = hidden_states.shape
        if hidden != H or router_logits.shape != (T, E):
            raise ValueError("hidden states [T, H] and router logits [T, E] must match the experts")
        if T == 0:
            return
        weights, _, sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_router(router_logits, top_k,
                                                                                    renormalize)
        self._experts(output, hidden_states, w1, w2, weights, top_k, sorted_routes, offsets, inverse)

    def _experts(self, output, hidden_states, w1, w2, topk_weights, topk, sorted_routes, offsets, inverse):
        E, H, I = self.shapes
        T = hidden_states.shape[0]
        routes = T * topk
        # Below ~96 routed rows per expert the grouped GEMMs stream each expert's weights
        # past its rows and produce their own MXFP8 operands (the activation quantization in
        # w13, the SwiGLU in w2) in LDS: route, w13, w2, combine -- four launches, the same
        # bits as the separate producers.
        if self.fuse and ops.grouped_fused_supported(routes, E, H, self.fmt) and hidden_states.stride(1) == 1:
            gate_up = torch.ops.mach_amd.grouped_gemm_quant(hidden_states, sorted_routes, topk, offsets, routes, w1,
                                                            self.w1_scale, 2 * I, H, self.fmt, self.act_rule)
        else:
            a, sa = torch.ops.mach_amd.quantize_mxfp8(hidden_states, self.act_rule)
            gate_up = torch.ops.mach_amd.grouped_gemm(a, sa, sorted_routes, topk, offsets, routes, w1,
                                                      self.w1_scale, 2 * I, H, self.fmt)
        swiglu_fused = self.fuse and ops.grouped_fused_supported(routes, E, I, self.fmt)
        if self.fuse_combine and ops.grouped_combine_supported(routes, E, H, I, self.fmt, swiglu_fused, topk) \
                and output.is_contiguous():
            # the weighted combine inside the down projection's launch (the same bits)
            if swiglu_fused:
                torch.ops.mach_amd.grouped_gemm_swiglu_combine(output, gate_up, offsets, routes, w2, self.w2_scale,
                                                               H, I, self.fmt, self.mid_rule, sorted_routes, inverse,
                                                               topk_weights)
            else:
                a2, sa2 = torch.ops.mach_amd.swiglu_mxfp8(gate_up, self.mid_rule, False)
                torch.ops.mach_amd.grouped_gemm_combine(output, a2, sa2, None, 1, offsets, routes, w2, self.w2_scale,
                                                        H, I, self.fmt, sorted_routes, inverse, topk_weights)
            return
        if swiglu_fused:
            y = torch.ops.mach_amd.grouped_gemm_swiglu(gate_up, offsets, routes, w2, self.w2_scale, H, I, self.fmt,
                                                       self.mid_rule)
        else:
            a2, sa2 = torch.ops.mach_amd.swiglu_mxfp8(gate_up, self.mid_rule, False)
            y = torch.ops.mach_amd.grouped_gemm(a2, sa2, None, 1, offsets, routes, w2, self.w2_scale, H, I, self.fmt)
        torch.ops.mach_amd.moe_reduce(output, y, topk_weights, inverse)

    def __call__(self, hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                 topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(hidden_states)
        self.apply(out, hidden_states, w1, w2, topk_weights, topk_ids, SILU, self.shapes[0], None,
                   None, None, None, None, None, False)
        return out


_MOE_PARAMS = ("w13_weight", "w13_weight_scale", "w2_weight", "w2_weight_scale")


def load_expert_shard(param: torch.nn.Parameter, loaded_weight: torch.Tensor, weight_name: str,
                      shard_id: str, expert_id: int) -> None:
    """vLLM's ``FusedMoE.weight_loader`` contract for one expert's tensor: shard ``w1`` (gate)
    fills rows [0, I) of expert ``expert_id``'s w13 entry, ``w3`` (up) rows [I, 2I), ``w2``
    (down) the whole w2 entry.  Shapes and dtypes must match exactly."""
    if not 0 <= expert_id < param.shape[0]:
        raise ValueError(f"expert {expert_id} is outside [0, {param.shape[0]})")
    target = param.data[expert_id]
    is_w13 = param.mxl_moe_name.startswith("w13")
    if shard_id in ("w1", "w3"):
        if not is_w13:
            raise ValueError(f"shard {shard_id} loads w13 parameters, not {param.mxl_moe_name}")
        half = target.shape[0] // 2
        target = target.narrow(0, 0 if shard_id == "w1" else half, half)
    elif shard_id == "w2":
        if is_w13:
            raise ValueError(f"shard w2 loads w2 parameters, not {param.mxl_moe_name}")
    else:
        raise ValueError(f"unknown expert shard {shard_id!r} (w1, w2 or w3)")
    if loaded_weight.dtype != target.dtype or tuple(loaded_weight.shape) != tuple(target.shape):
        raise ValueError(f"{weight_name}: checkpoint tensor {loaded_weight.dtype}{tuple(loaded_weight.shape)} "
                         f"does not match {target.dtype}{tuple(target.shape)}")
    target.copy_(loaded_weight)


class Mxfp6MoEMethod:
    """``FusedMoEMethodBase``-shaped owner of routed-expert MXFP6 parameters.

    ``create_weights`` registers the Quark OCP-MX checkpoint layout that the reference's
    patched ``QuarkOCP_MX_MoEMethod`` loads (src/vllm_mach/mxfp6/profile/runtime.patch:207-250):
    ``w13_weight`` u8 [E, 2I, 3H/4], ``w13_weight_scale`` u8 [E, 2I, H/32], ``w2_weight``
    u8 [E, H, 3I/4], ``w2_weight_scale`` u8 [E, H, I/32], each with vLLM's
    ``weight_loader(param, loaded_weight, weight_name, shard_id, expert_id)``.
    ``process_weights_after_loading`` replaces them with the MFMA-tiled layout (where the
    reference repacks scales, runtime.patch:227-239), and ``apply`` routes and runs them.
    H and I must be multiples of 128 (the tiled layout's K granule).
    """

    def __init__(self, fmt: int = ops.E3M2, act_rule: int = ops.FLOOR_CARRY175,
                 mid_rule: int = ops.CEIL_DIV448):
        if fmt not in (ops.E2M3, ops.E3M2):
            raise ValueError("MXFP6 MoE weights are E2M3 or E3M2")
        self.experts = Mxfp6Experts(fmt, act_rule, mid_rule)

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype,
                       **extra_weight_attrs) -> None:
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        if E <= 0 or H <= 0 or I <= 0 or H % 128 or I % 128:
            raise ValueError("MXFP6 MoE needs experts > 0 and hidden and intermediate sizes divisible by 128")
        attrs = dict(extra_weight_attrs)
        device = attrs.pop("device", None)
        shapes = ((E, 2 * I, H * 3 // 4), (E, 2 * I, H // 32), (E, H, I * 3 // 4), (E, H, I // 32))
        for name, shape in zip(_MOE_PARAMS, shapes):
            param = torch.nn.Parameter(torch.empty(shape, dtype=torch.uint8, device=device), requires_grad=False)
            param.mxl_moe_name = name
            param.weight_loader = load_expert_shard
            for attr, value in attrs.items():
                setattr(param, attr, value)
            layer.register_parameter(name, param)
        layer.params_dtype = params_dtype
        layer.local_num_experts = E

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        w1, w2 = self.experts.process_weights_after_loading(
            layer.w13_weight.data, layer.w13_weight_scale.data, layer.w2_weight.data, layer.w2_weight_scale.data)
        for name, value in zip(_MOE_PARAMS, (w1, self.experts.w1_scale, w2, self.experts.w2_scale)):
            setattr(layer, name, torch.nn.Parameter(value, requires_grad=False))
        layer.mxl_experts = self.experts  # found by warmup()

    def apply_router(self, layer: torch.nn.Module, x: torch.Tensor, router_logits: torch.Tensor,
                     top_k: int, renormalize: bool = True) -> torch.Tensor:
        """The layer from router logits (``Mxfp6Experts.apply_router``): routing fused
        ahead of the expert GEMMs, as the reference's MoE runner does
        (src/vllm_mach/mxfp6/moe.py:219-240)."""
        out = torch.empty_like(x)
        self.experts.apply_router(out, x, layer.w13_weight, layer.w2_weight, router_logits, top_k, renormalize)
        return out

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, topk_weights: torch.Tensor,
              topk_ids: torch.Tensor, expert_map: Optional[torch.Tensor] = None,
              global_num_experts: Optional[int] = None) -> torch.Tensor:
        out = torch.empty_like(x)
        E = self.experts.shapes[0] if self.experts.shapes is not None else layer.local_num_experts
        self.experts.apply(out, x, layer.w13_weight, layer.w2_weight, topk_weights, topk_ids, SILU,
                           E if global_num_experts is None else global_num_experts, expert_map,
                           None, None, None, None, None, False)
        return out
