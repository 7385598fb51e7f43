"""MXFP6 (W6A8) routed-expert MoE on MI355X.

``Mxfp6Experts.apply`` keeps the signature and mutation contract of the
reference's ``Mxfp6Sm120Experts.apply`` (src/vllm_mach/mxfp6/moe.py:574-702):
quantize hidden states to MXFP8 -> stable token sort by expert -> grouped
W6A8 GEMM (w13) -> SwiGLU (bf16 SiLU) + MXFP8 -> grouped W6A8 GEMM (w2) ->
fp32 weighted combine into ``output``.  The grouped GEMMs gather activation
rows through the sorted route list, so no permuted copy of the activations is
written, and experts that receive no rows read no weights.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops

SILU = "silu"


def select_experts(router_logits: torch.Tensor, top_k: int, renormalize: bool = True):
    """softmax -> top-k -> optional renormalization (fp32 weights, int32 ids)."""
    probs = torch.softmax(router_logits.float(), dim=-1)
    weights, ids = torch.topk(probs, top_k, dim=-1)
    if renormalize:
        weights = weights / weights.sum(dim=-1, keepdim=True)
    return weights.float(), ids.to(torch.int32)


class Mxfp6Experts:
    """Routed experts over packed MXFP6 weights.

    Checkpoint layout (Quark OCP-MX): w13 u8 [E, 2I, 3H/4] + E8M0 [E, 2I, H/32] (gate rows
    [0, I), up rows [I, 2I)); w2 u8 [E, H, 3I/4] + E8M0 [E, H, I/32].
    """

    def __init__(self, fmt: int = ops.E2M3, act_rule: int = ops.FLOOR_CARRY175,
                 mid_rule: int = ops.CEIL_DIV448):
        self.fmt = fmt
        self.act_rule = act_rule
        self.mid_rule = mid_rule
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
        a, sa = torch.ops.mach_amd.quantize_mxfp8(hidden_states, self.act_rule)
        sorted_routes, offsets, inverse = torch.ops.mach_amd.moe_route(ids, E)
        routes = T * topk
        gate_up = torch.ops.mach_amd.grouped_gemm(a, sa, sorted_routes, topk, offsets, routes, w1,
                                                  self.w1_scale, 2 * I, H, self.fmt)
        a2, sa2 = torch.ops.mach_amd.swiglu_mxfp8(gate_up, self.mid_rule, False)
        y = torch.ops.mach_amd.grouped_gemm(a2, sa2, None, 1, offsets, routes, w2, self.w2_scale, H, I, self.fmt)
        torch.ops.mach_amd.moe_reduce(output, y, topk_weights, inverse)

    def __call__(self, hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                 topk_weights: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(hidden_states)
        self.apply(out, hidden_states, w1, w2, topk_weights, topk_ids, SILU, self.shapes[0], None,
                   None, None, None, None, None, False)
        return out
