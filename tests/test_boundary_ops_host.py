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
    # the two-limb path's operator, checked when dual dispatch is enabled (native_backend.py:90-93)
    "dual_gemm_out": ("Tensor hi", "Tensor weight", "Tensor s_hi", "Tensor s_weight", "Tensor res",
                      "Tensor s_res", "Tensor(a!) out"),
}
# src/vllm_mach/moe_utils.py:15-26: the names is_mxfp6_sm120_available() requires of the package
MXFP6_REQUIRED_API = ("MXFP8Tensor", "PackedMXFP6Tensor", "autotune_w6a8", "begin_workspace_planning",
                      "finalize_workspace_planning", "gemm_w6a8", "is_available", "load_library", "pack_scales",
                      "workspace_stats")


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
    # the PDL entry points _require_pdl_runtime() looks for (dense_mxfp8.py:63-67)
    for name in ("gemm_pdl", "gemm_from_float_pdl"):
        assert hasattr(torch.ops.mxfp8_sm120, name), name
    assert hasattr(torch.ops.mxfp6, "quantize_mxfp8_pdl")
    assert str(torch.ops.mxfp8_sm120.gemm_from_float_pdl.default._schema) == \
        "mxfp8_sm120::gemm_from_float_pdl(Tensor x, Tensor w, Tensor ws) -> Tensor"


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


def test_dense_api_and_runtime_modules(loaded):
    """The package names the reference's availability check requires (moe_utils.py:15-26,
    139-146), the dense MXFP8 runtime module's names (dense_mxfp8.py:120-125, 151) and the
    two-limb module's (mxfp8/dual.py:42-45, 109-111)."""
    for name in MXFP6_REQUIRED_API + ("gemm_from_float", "warmup_w6a8", "quantize_mxfp8"):
        assert hasattr(loaded, name), name
    for name in ("load_library", "gemm_from_float", "begin_workspace_planning", "finalize_workspace_planning",
                 "warmup", "MXFP8Tensor", "pack_scales"):
        assert hasattr(loaded.mxfp8, name), name
    for name in ("load_library", "quantize", "gemm_out"):
        assert hasattr(loaded.mxfp8_dual, name), name
    t = loaded.PackedMXFP6Tensor(values=torch.zeros(8, 96, dtype=torch.uint8), scales=torch.zeros(4),
                                 rows=8, k=128)
    assert (t.rows, t.k) == (8, 128)
    assert loaded.MXFP8Tensor(torch.zeros(2, 32), torch.zeros(4), 2, 32).k == 32
