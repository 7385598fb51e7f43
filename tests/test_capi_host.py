"""CPU checks of the boundary: the C ABI library loads and exports every symbol the
header declares (no compute calls without a GPU), the Python binding matches the
header, argument validation fails closed, and the host-side contracts of the
reference's kernel classes hold (admission rules, symbolic fakes, capture-miss
errors, loud failure without the library)."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mxlinear.h"
LIB = ROOT / "vllm-mach_amd" / "libmxlinear.so"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(mxl_[a-z0-9_]+)\s*\(", text))


def test_header_symbols_exported():
    if not LIB.exists():
        pytest.skip("libmxlinear.so not built")
    lib = ctypes.CDLL(str(LIB))
    names = _declared()
    assert len(names) >= 17
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_matches_header(pkg):
    from vllm_mach_amd import _lib
    assert set(_lib.SIGNATURES) == _declared()


def test_pure_queries_without_gpu(pkg):
    from vllm_mach_amd import _lib
    if not LIB.exists():
        pytest.skip("libmxlinear.so not built")
    assert _lib.query("mxl_version") >= 1
    assert _lib.query("mxl_tiled_weight_bytes", 2048, 2048, 0) == 128 * 4 * 8 * 1024
    assert _lib.query("mxl_tiled_weight_bytes", 17408, 5120, 2) == 1088 * 10 * 6 * 1024
    assert _lib.query("mxl_tiled_scale_bytes", 16, 1024) == 2 * 256
    assert _lib.query("mxl_swizzled_scale_bytes", 1, 9216) == 128 * 72 * 4
    assert _lib.query("mxl_moe_route_workspace_bytes", 2048, 8, 256) == 16 * 256 * 4


def test_invalid_arguments_fail_before_any_launch(pkg):
    """Argument checks return MXL_EINVAL with a message; nothing reaches HIP."""
    from vllm_mach_amd import _lib
    if not LIB.exists():
        pytest.skip("libmxlinear.so not built")
    with pytest.raises(_lib.MxlError, match="K % 32"):
        _lib.call("mxl_quantize_mxfp8", 16, 4, 33, 33, 0, 16, 16, None)
    with pytest.raises(_lib.MxlError, match="unknown rule"):
        _lib.call("mxl_quantize_mxfp8", 16, 4, 64, 64, 7, 16, 16, None)
    with pytest.raises(_lib.MxlError, match="unknown weight format"):
        _lib.call("mxl_mx_gemm", 16, 16, 1, 16, 16, 16, 128, 1, None, 16, 16, None, 0, None)
    with pytest.raises(_lib.MxlError, match="K % 128"):
        _lib.call("mxl_pack_weight", 16, 16, 16, 100, 0, 16, 16, None)
    with pytest.raises(_lib.MxlError, match="workspace too small"):
        _lib.call("mxl_moe_route", 16, 4096, 8, 256, 16, 16, 16, None, 0, None)


def test_missing_library_fails_loudly(tmp_path, monkeypatch, pkg):
    from vllm_mach_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.lib()


def test_mxfp6_admission_rules(pkg):
    from vllm_mach_amd.linear import logical_mxfp6_shape
    assert logical_mxfp6_shape(torch.empty(17408, 3840, dtype=torch.uint8)) == (17408, 5120)
    for shape, msg in [((8, 97), "three bytes"), ((12, 96), "N % 8"), ((8, 72), "K % 128")]:
        with pytest.raises(ValueError, match=msg):
            logical_mxfp6_shape(torch.empty(*shape, dtype=torch.uint8))
    with pytest.raises(ValueError, match="two-dimensional"):
        logical_mxfp6_shape(torch.empty(2, 8, 96, dtype=torch.uint8))


def test_kernel_selection_contract(pkg):
    from vllm_mach_amd import linear as L
    ok, _ = L.Mxfp6LinearKernel.can_implement(L.MxLinearLayerConfig(L.MXFP6_E3M2_STATIC, L.MXFP8_DYNAMIC))
    assert ok
    ok, why = L.Mxfp6LinearKernel.can_implement(L.MxLinearLayerConfig(L.MXFP8_STATIC, L.MXFP8_DYNAMIC))
    assert not ok and "MXFP6" in why
    ok, why = L.Mxfp6LinearKernel.can_implement(L.MxLinearLayerConfig(L.MXFP6_E2M3_STATIC, "fp8_static"))
    assert not ok and "dynamic MXFP8" in why
    reg = L.register_kernels({"mxfp8": [object], "mxfp6": [L.Mxfp6LinearKernel, object]})
    assert reg["mxfp8"][0] is L.Mxfp8LinearKernel and reg["mxfp6"] == [L.Mxfp6LinearKernel, object]
    if not torch.cuda.is_available():
        ok, why = L.Mxfp8LinearKernel.is_supported()
        assert not ok and why


def test_create_weights_checkpoint_layouts(pkg):
    from vllm_mach_amd import linear as L
    for key, wshape, sname, sshape, sdtype in [
        (L.MXFP8_STATIC, (384, 256), "weight_scale", (384, 8), torch.uint8),
        (L.MXFP6_E2M3_STATIC, (384, 192), "weight_scale", (384, 8), torch.uint8),
        (L.FP8_BLOCK128, (384, 256), "weight_scale_inv", (3, 2), torch.float32),
    ]:
        layer = torch.nn.Module()
        L.MxLinearMethod(key).create_weights(layer, 256, [128, 256], 256, 384, torch.bfloat16)
        assert tuple(layer.weight.shape) == wshape
        s = getattr(layer, sname)
        assert tuple(s.shape) == sshape and s.dtype == sdtype
        assert layer.logical_widths == [128, 256]


def test_fake_impls_keep_rows_symbolic(pkg):
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.symbolic_shapes import ShapeEnv
    mode = FakeTensorMode(shape_env=ShapeEnv())
    with mode:
        x = mode.from_tensor(torch.empty(16, 2048, dtype=torch.bfloat16),
                             symbolic_context=None)
    # mark the row dimension dynamic through a real compile-time trace
    def f(x, w, sw):
        a, sa = torch.ops.mach_amd.quantize_mxfp8(x, 0)
        return torch.ops.mach_amd.mx_gemm(a, sa, w, sw, 256, 2048, 0, None)
    from torch.fx.experimental.proxy_tensor import make_fx
    gm = make_fx(f, tracing_mode="symbolic")(torch.empty(16, 2048, dtype=torch.bfloat16),
                                             torch.empty(10, dtype=torch.uint8), torch.empty(4, dtype=torch.uint8))
    outs = [n for n in gm.graph.nodes if n.op == "call_function" and "mx_gemm" in str(n.target)]
    assert outs
    val = outs[0].meta["val"]
    assert isinstance(val.shape[0], torch.SymInt) and val.shape[1] == 256


def test_workspace_capture_miss_raises(pkg, monkeypatch):
    from vllm_mach_amd import ops
    monkeypatch.setattr(ops, "stream_handle", lambda device: 0x1234)
    monkeypatch.setattr(ops, "_workspaces", {})
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    cpu = torch.device("cpu")
    buf = ops.workspace(cpu, 100)
    assert buf.numel() >= 100 and ops.workspace(cpu, 50) is buf
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert ops.workspace(cpu, 80) is buf
    with pytest.raises(RuntimeError, match="before graph capture"):
        ops.workspace(cpu, 10_000)
