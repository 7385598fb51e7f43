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
    # the scatter's per-wavefront histograms bound the expert count (160 KiB of LDS)
    with pytest.raises(_lib.MxlError, match="at most 2560 experts"):
        _lib.call("mxl_moe_route", 16, 4096, 8, 2561, 16, 16, 16, 16, 1 << 30, None)
    # mxl_gemm_options fields outside their ranges are argument errors, not defaults
    for bad in ({"tile_n": 3}, {"tile_m": 2}, {"waves": 6}, {"hybrid": 2}, {"kernel": 9}, {"sa_layout": 2}):
        opts = _lib.GemmOptions(**bad)
        with pytest.raises(_lib.MxlError, match="sa_layout|invalid options|unknown"):
            _lib.call("mxl_mx_gemm_ex", 16, 16, 1, 16, 16, 16, 128, 0, None, 16, 16, None, 0,
                      _lib.options_ptr(opts), None)
    with pytest.raises(_lib.MxlError, match="invalid options"):
        _lib.call("mxl_mx_gemm_dual_ex", 16, 16, 16, 16, 1, 16, 16, 16, 128, 0, None, 16, 16, 16, 1 << 20,
                  _lib.options_ptr(_lib.GemmOptions(waves=5)), None)
    # the output scale and format: a zero-filled struct (alpha 0) is refused, as are unknown
    # formats and non-finite scales; the grouped and two-limb GEMMs write bf16 unscaled only
    for bad in ({"alpha": 0.0}, {"alpha": float("inf")}, {"alpha": float("nan")}, {"out_dtype": 2}):
        opts = _lib.GemmOptions(**bad)
        with pytest.raises(_lib.MxlError, match="alpha must be finite"):
            _lib.call("mxl_mx_gemm_ex", 16, 16, 1, 16, 16, 16, 128, 0, None, 16, 16, None, 0,
                      _lib.options_ptr(opts), None)
        with pytest.raises(_lib.MxlError, match="invalid"):
            _lib.call("mxl_quant_mx_gemm_ex", 16, 1, 128, 0, 16, 16, 16, 0, None, 16, 16,
                      _lib.options_ptr(opts), None)
    with pytest.raises(_lib.MxlError, match="bf16 output without scaling only"):
        _lib.call("mxl_grouped_gemm_ex", 16, 16, 16, None, 1, 16, 1, 16, 16, 16, 16, 128, 0, 16,
                  _lib.options_ptr(_lib.GemmOptions(out_dtype=1)), None)
    with pytest.raises(_lib.MxlError, match="bf16 output without scaling only"):
        _lib.call("mxl_mx_gemm_dual_ex", 16, 16, 16, 16, 1, 16, 16, 16, 128, 0, None, 16, 16, 16, 1 << 20,
                  _lib.options_ptr(_lib.GemmOptions(alpha=0.5)), None)


def test_plan_names_without_gpu(pkg):
    """The kernels a call launches, as the profiler names them: what the committed traffic
    rows and traces are matched against.  (No GPU here: the plan assumes 256 CUs.)"""
    from vllm_mach_amd import _lib
    if not LIB.exists():
        pytest.skip("libmxlinear.so not built")
    if torch.cuda.is_available():
        pytest.skip("the expected plans are those of a 256-CU device")
    name = lambda *a, **k: _lib.plan_name("mxl_gemm_plan_name", *a, **k)  # noqa: E731
    assert name(16, 2560, 9216, 0, 0) == "gemm_stream_kernel<0,2,false,false,-1,-1>"
    assert name(16, 2048, 2048, 0, 0) == "gemm_stream_kernel<0,1,true,false,-1,-1>"
    # c2 M = 512: 128 x 128 tiles, three K splits, eight waves
    assert name(512, 2560, 9216, 0, 0) == "gemm_wide_kernel<0,8,2,false,false,2> + wide_tile_reduce_kernel"
    assert name(512, 2560, 9216, 0, 0, options=_lib.GemmOptions(waves=4)) == \
        "gemm_wide_kernel<0,8,2,false,false,1> + wide_tile_reduce_kernel"
    wide8 = name(512, 2560, 9216, 0, 0, options=_lib.GemmOptions(waves=8))
    assert wide8.startswith("gemm_wide_kernel<0,8,") and wide8.split(" + ")[0].endswith(",2>")
    assert name(40, 1024, 1024, 3, 0).startswith("gemm_kernel<3,")
    assert name(512, 2560, 9216, 0, 0, options=_lib.GemmOptions(tile_n=2, splits=3)) == \
        "gemm_wide_kernel<0,8,2,false,false,1> + wide_tile_reduce_kernel"
    # block-FP8 prefill at c3 (N = 18432, K = 2560): eight waves on 128 x 128 tiles, the
    # remainder split only when one full round precedes it
    assert name(128, 18432, 2560, 0, 1) == "gemm_wide_kernel<0,8,2,true,false,2>"
    assert name(256, 18432, 2560, 0, 1) == "gemm_wide_kernel<0,8,2,true,false,2> + wide_tile_reduce_kernel"
    assert name(512, 18432, 2560, 0, 1) == "gemm_wide_kernel<0,8,2,true,false,2>"
    assert name(512, 18432, 2560, 0, 1, options=_lib.GemmOptions(waves=4)).split(" + ")[0].endswith(",1>")
    grouped = lambda *a: _lib.plan_name("mxl_grouped_plan_name", *a)  # noqa: E731
    assert grouped(1024, 256, 2048, 2, 1, 0) == "gemm_stream_grouped_kernel<2,1,4>"
    assert grouped(1024, 256, 512, 2, 2, 1) == "gemm_stream_grouped_kernel<2,1,9>"
    assert grouped(16384, 256, 512, 2, 0, 0) == "gemm_stream_grouped_kernel<2,6,0>"
    assert grouped(16384, 256, 2048, 2, 0, 0) == "gemm_wide_kernel<2,8,2,false,true,1>"


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
    monkeypatch.setattr(ops, "_planned", {})
    monkeypatch.setattr(ops, "_retired", [])
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    cpu = torch.device("cpu", 0)
    buf = ops.workspace(cpu, 100)
    assert buf.numel() >= 100 and ops.workspace(cpu, 50) is buf
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert ops.workspace(cpu, 80) is buf
    with pytest.raises(RuntimeError, match="before graph capture"):
        ops.workspace(cpu, 10_000)


def test_workspace_growth_keeps_captured_buffers(pkg, monkeypatch):
    """A buffer handed to a call during capture stays alive after a larger shape replaces
    it (a captured graph writes through its address on replay); one never captured is
    released."""
    from vllm_mach_amd import ops
    monkeypatch.setattr(ops, "stream_handle", lambda device: 0x77)
    monkeypatch.setattr(ops, "_workspaces", {})
    monkeypatch.setattr(ops, "_planned", {})
    monkeypatch.setattr(ops, "_retired", [])
    cpu = torch.device("cpu", 0)
    capturing = [False]
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: capturing[0])
    a = ops.workspace(cpu, 1000)
    b = ops.workspace(cpu, 5000)          # grows: a was never captured, so it is not kept
    assert b is not a and ops._retired == []
    capturing[0] = True
    assert ops.workspace(cpu, 4000) is b  # a graph now holds b's address
    capturing[0] = False
    c = ops.workspace(cpu, 20000)
    assert c is not b and len(ops._retired) == 1 and ops._retired[0] is b
    assert c.numel() >= 20000
    info = ops.inspect()
    assert info["workspaces"] == {"0:0x77:gemm": c.numel()}
    assert info["planned"] == {"0:gemm": 20000} and info["retired_bytes"] == b.numel()


def test_reserve_workspaces_sizes_a_new_stream(pkg, monkeypatch):
    from vllm_mach_amd import ops
    stream = [0x10]
    monkeypatch.setattr(ops, "stream_handle", lambda device: stream[0])
    monkeypatch.setattr(ops, "_workspaces", {})
    monkeypatch.setattr(ops, "_planned", {})
    monkeypatch.setattr(ops, "_retired", [])
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    cpu = torch.device("cpu", 0)
    ops.workspace(cpu, 300, "gemm")
    ops.workspace(cpu, 9000, "gemm")
    ops.workspace(cpu, 64, "route")
    stream[0] = 0x20                       # the capture stream
    ops.reserve_workspaces(cpu)
    ws = ops.inspect()["workspaces"]
    assert ws["0:0x20:gemm"] >= 9000 and ws["0:0x20:route"] >= 64
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    assert ops.workspace(cpu, 9000, "gemm").numel() >= 9000   # no allocation during capture


def test_warmup_collects_distinct_problems(pkg):
    from vllm_mach_amd import linear as L, warmup as W
    layers = []
    for n in (256, 256, 384):
        layer = torch.nn.Module()
        layer.mxl_shape = (n, 512)
        layer.mxl_format = 0
        layer.mxl_kernel = L.Mxfp8LinearKernel()
        layers.append(layer)
    dense, moe = W.collect_problems(layers)
    assert sorted((k[1], k[2]) for k in dense) == [(256, 512), (384, 512)] and moe == {}
    assert W._sizes([1, 16, 300]) == [300, 256, 128, 64, 16, 1]
    assert W._sizes([]) == []
