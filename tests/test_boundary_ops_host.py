"""CPU checks of the reference-named torch operator library (``libmxlinear_torch.so``):
it loads with ``torch.ops.load_library`` and registers exactly the schemas the
reference's loaders verify before binding (no GPU work)."""
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "vllm-mach_amd" / "libmxlinear_torch.so"

# src/vllm_mach/fp8/block_native.py:15 compares the whole string
BLOCK_FP8_SCHEMA = "vllm_mach_block_fp8::mm(Tensor a, Tensor b, Tensor sa, Tensor sb) -> Tensor"
# native/fp8_activation/activation.cu:99-100 (the definition the reference's adapter calls)
ACTIVATION_SCHEMA = ("mach_fp8_activation::run(Tensor(a!) out, Tensor input, Tensor(b!) scales, "
                     "bool is_scale_transposed) -> ()")
# src/vllm_mach/mxfp8/native_backend.py:77-97: fragments every schema must contain
MXFP8_FRAGMENTS = {
    "gemm": ("Tensor a", "Tensor b", "Tensor sa", "Tensor sb", "Tensor(a!)? out", "Tensor? workspace",
             "int tactic", "int splits", "int swizzle", "int sms"),
    "allocate_workspace": ("Tensor a", "Tensor b", "Tensor sa", "Tensor sb", "Tensor out", "int tactic",
                           "int splits", "int swizzle", "int sms"),
}


@pytest.fixture(scope="module")
def loaded(pkg):
    if not LIB.exists():
        pytest.skip("libmxlinear_torch.so not built")
    from vllm_mach_amd import mxfp6_api
    assert mxfp6_api.load_library() == str(LIB)
    return mxfp6_api


def test_block_fp8_and_activation_schemas_exact(loaded):
    assert str(torch.ops.vllm_mach_block_fp8.mm.default._schema) == BLOCK_FP8_SCHEMA
    assert str(torch.ops.mach_fp8_activation.run.default._schema) == ACTIVATION_SCHEMA


def test_mxfp8_schema_fragments(loaded):
    for name, fragments in MXFP8_FRAGMENTS.items():
        schema = str(getattr(torch.ops.mxfp8_sm120, name).default._schema)
        assert all(f in schema for f in fragments), schema
    # the PDL-capable ABI test of src/vllm_mach/mxfp6/dense_mxfp8.py:58-65
    assert "bool use_pdl=False" in str(torch.ops.mxfp8_sm120.gemm.default._schema)
    assert "mxfp8_sm120::gemm_from_float(Tensor x, Tensor w, Tensor ws) -> Tensor" == \
        str(torch.ops.mxfp8_sm120.gemm_from_float.default._schema)


def test_mxfp6_op_signatures(loaded):
    """Argument lists of the mxfp6 ops at their call sites (dense.py:122-129 (x, w, ws, N,
    alpha, dtype); fused_mlp.py:18-19; ar_norm.py:145-147 (codes, w, scales, ws, M, N, K,
    alpha, dtype); dense_mxfp8.py:40 quantize_mxfp8(x) -> (codes, scales))."""
    ops = torch.ops.mxfp6
    args = lambda op: [a.name for a in op.default._schema.arguments]
    assert args(ops.gemm_from_float) == ["x", "w", "ws", "N", "alpha", "dtype"]
    assert args(ops.gemm_from_swiglu) == ["gate_up", "w", "ws", "N", "alpha", "dtype"]
    assert args(ops.gemm_w6a8_pdl) == ["codes", "w", "scales", "ws", "M", "N", "K", "alpha", "dtype"]
    assert args(ops.quantize_mxfp8) == ["x"] and len(ops.quantize_mxfp8.default._schema.returns) == 2
    assert args(ops.pack_scales) == ["scales"]


def test_moe_api_names(loaded):
    """The mxfp6 package API the reference's MoE path calls (moe_utils.py:15-44, 162-488)."""
    for name in ("quantize_mxfp8_logical", "quantize_mxfp8", "pack_scales", "to_mma_k64_weight",
                 "route_mxfp8_out", "grouped_gemm_w6a8_out", "silu_and_mul_mxfp8_grouped", "moe_reduce_out",
                 "begin_workspace_planning", "finalize_workspace_planning", "workspace_stats", "load_library",
                 "is_available"):
        assert callable(getattr(loaded, name)), name
    if not torch.cuda.is_available():
        assert loaded.is_available() is False
