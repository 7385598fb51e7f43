"""HIP graph capture after warmup, and the capture contract of the reference-named ops.

* ``warmup.warmup`` (the reference's ``warmup_mxfp8`` / ``warmup_mxfp6_sm120(_stream)``,
  src/vllm_mach/mxfp6/dense_mxfp8.py:177-220, src/vllm_mach/mxfp6/warmup.py:75-147) on a
  model holding one layer of each dense kernel and one routed-expert layer, then the
  capture-stream registration, then a capture at every warmed size: no workspace is
  allocated or replaced during capture, and every replay equals the eager result bit for bit.
* ``libmxlinear_torch.so`` (``mxfp8_sm120::gemm``, native_backend.py:159-205): a capture
  on a stream whose workspace was not warmed for the shape raises instead of running with
  less scratch; once warmed, the replay equals the eager result bit for bit.
* The torch op library's tiled-weight cache drops the copy of a freed weight.
"""
import warnings

import numpy as np
import pytest
import torch

from test_gpu_gemm import _act, _weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def api(pkg):
    from vllm_mach_amd import mxfp6_api
    mxfp6_api.load_library()
    return mxfp6_api


def _replay_matches(graph, stream, outs, eager):
    for _ in range(3):
        graph.replay()
        stream.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)


def test_mxfp8_sm120_gemm_capture_needs_warm_stream(api, oracle_mod, dev):
    """c2 at M = 512 (a K-split plan): unwarmed capture stream raises, warmed replays match."""
    M, N, K = 512, 2560, 9216
    wc, ws, _ = _weights(oracle_mod, N, K, 0, 0.02, 23)
    b = torch.from_numpy(wc).to(dev).view(torch.float8_e4m3fn)
    sb = api.pack_scales(torch.from_numpy(ws).to(dev))
    x = _act(M, K, 31).to(dev)
    codes, sa = torch.ops.mxfp6.quantize_mxfp8(x)
    a = codes.view(torch.float8_e4m3fn)
    torch.ops.mxfp8_sm120.gemm(a[:16], b, sa, sb)  # the weight's tiled copy exists (no workspace at M = 16)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream), warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="The CUDA Graph is empty")
        g0 = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="warm this shape before capture"):
            with torch.cuda.graph(g0, stream=stream):
                torch.ops.mxfp8_sm120.gemm(a, b, sa, sb)
    with torch.cuda.stream(stream):
        eager = torch.ops.mxfp8_sm120.gemm(a, b, sa, sb)  # warms this stream's workspace
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = torch.ops.mxfp8_sm120.gemm(a, b, sa, sb)
        _replay_matches(graph, stream, [out], [eager])
        assert torch.equal(torch.ops.mxfp8_sm120.gemm(a, b, sa, sb), eager)
    torch.cuda.current_stream().wait_stream(stream)


def test_tiled_copy_of_freed_weight_is_released(api, oracle_mod, dev):
    """A weight's MFMA-tiled copy lives while the weight does: after the weight is freed the
    next calls of the op library drop it, and device memory returns to its level before."""
    M, N, K = 4, 4096, 4096
    wc, ws, _ = _weights(oracle_mod, N, K, 0, 0.02, 5)
    keep = torch.from_numpy(wc).to(dev).view(torch.float8_e4m3fn)
    keep_s = api.pack_scales(torch.from_numpy(ws).to(dev))
    x = _act(M, K, 3).to(dev)
    torch.ops.mxfp8_sm120.gemm_from_float(x, keep, keep_s)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    for _ in range(3):  # each time a new weight (its own tiled copy, about 16.5 MB)
        w = keep.clone()
        s = keep_s.clone()
        torch.ops.mxfp8_sm120.gemm_from_float(x, w, s)
        torch.cuda.synchronize()
        grown = torch.cuda.memory_allocated(dev) - base
        assert grown >= 2 * N * K, grown  # the weight and its tiled copy
        del w, s
        for _ in range(4):  # calls on the kept weight sweep the cache
            torch.ops.mxfp8_sm120.gemm_from_float(x, keep, keep_s)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated(dev) == base


def _dense_layer(pkg, dev, key, N, K, seed):
    L = pkg.linear
    g = torch.Generator().manual_seed(seed)
    layer = torch.nn.Module()
    method = L.MxLinearMethod(key)
    method.create_weights(layer, K, [N], K, N, torch.bfloat16, device=dev)
    w = (torch.randn(N, K, generator=g) * 0.02).bfloat16().to(dev)
    if key == L.MXFP8_STATIC:
        codes, scales = torch.ops.mach_amd.quantize_mxfp8(w, 0)
        layer.weight.data.copy_(codes)
        layer.weight_scale.data.copy_(scales)
    elif key == L.FP8_BLOCK128:
        wb = w.float().reshape(N // 128, 128, K // 128, 128)
        sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
        layer.weight.data.copy_((wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn))
        layer.weight_scale_inv.data.copy_(sb)
    else:
        packed, scales = torch.ops.mach_amd.quantize_mxfp6(w, 3 if key == L.MXFP6_E3M2_STATIC else 2)
        layer.weight.data.copy_(packed)
        layer.weight_scale.data.copy_(scales)
    method.process_weights_after_loading(layer)
    layer.method = method
    return layer


def _moe_layer(pkg, dev, E, H, I, seed):
    g = torch.Generator().manual_seed(seed)
    layer = torch.nn.Module()
    method = pkg.moe.Mxfp6MoEMethod(fmt=2)
    method.create_weights(layer, E, H, I, torch.bfloat16, device=dev)
    for name, (n, k) in (("w13", (2 * I, H)), ("w2", (H, I))):
        w = (torch.randn(E * n, k, generator=g) * 0.05).bfloat16().to(dev)
        packed, scales = torch.ops.mach_amd.quantize_mxfp6(w, 2)
        getattr(layer, f"{name}_weight").data.copy_(packed.view(E, n, k * 3 // 4))
        getattr(layer, f"{name}_weight_scale").data.copy_(scales.view(E, n, k // 32))
    method.process_weights_after_loading(layer)
    layer.method = method
    layer.top_k = 8
    return layer


def test_warmup_then_capture_allocates_no_workspace(pkg, dev):
    """warmup(model, sizes), then warmup(model, sizes, stream=True) on the capture stream,
    then one graph per size over every layer: the workspace table and the miss counters do
    not change during the captures, and each replay equals the eager pass bit for bit."""
    ops, L, warmup = pkg.ops, pkg.linear, pkg.warmup
    dense = [_dense_layer(pkg, dev, L.MXFP8_STATIC, 2560, 9216, 1),
             _dense_layer(pkg, dev, L.MXFP6_E2M3_STATIC, 4352, 5120, 2),
             _dense_layer(pkg, dev, L.FP8_BLOCK128, 4608, 2560, 3)]
    moe = _moe_layer(pkg, dev, 32, 1024, 512, 4)
    model = torch.nn.ModuleList(dense + [moe])
    sizes = [1, 16, 128, 512]
    report = warmup.warmup(model, sizes)
    assert len(report["dense"]) == 3 and len(report["moe"]) == 1
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    gen = torch.Generator().manual_seed(9)
    with torch.cuda.stream(stream):
        warmup.warmup(model, sizes, stream=True)
        stream.synchronize()
        before = ops.inspect()
        for m in sizes:
            xs = [torch.randn(m, layer.mxl_shape[1], generator=gen).bfloat16().to(dev) for layer in dense]
            xm = torch.randn(m, 1024, generator=gen).bfloat16().to(dev)
            logits = torch.randn(m, 32, generator=gen).to(dev)
            wts, ids = pkg.moe.select_experts(logits, 8)

            def run():
                ys = [layer.method.apply(layer, x) for layer, x in zip(dense, xs)]
                ys.append(moe.method.apply(moe, xm, wts, ids))
                return ys

            eager = run()
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                outs = run()
            _replay_matches(graph, stream, outs, eager)
        after = ops.inspect()
    torch.cuda.current_stream().wait_stream(stream)
    assert after["workspaces"] == before["workspaces"]
    assert after["retired_bytes"] == before["retired_bytes"]
    assert after["counts"].get("workspace_miss", 0) == before["counts"].get("workspace_miss", 0)
    assert "capture_cache_miss" not in after["counts"]
