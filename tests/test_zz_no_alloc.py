"""The no-allocation GEMM entry point (mxl_mx_gemm_noalloc) against mxl_mx_gemm with a
workspace, through the C ABI: same plan, so the same bits, on consecutive calls whose
second is smaller (the library-owned scratch keeps the first call's partials); against
the oracle; and the clear error for a shape whose split needs more scratch than it holds."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import _act, _check, _weights

pytestmark = pytest.mark.gpu


def _case(pkg, oracle_mod, dev, M, N, K, fmt, seed):
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, seed)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, seed + 1)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    return wc, ws, x, a, sa, tiled, tiled_s


def _noalloc(pkg, a, sa, tiled, tiled_s, M, N, K, fmt, bias=None):
    from vllm_mach_amd import _lib
    out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _lib.call("mxl_mx_gemm_noalloc", a.data_ptr(), sa.data_ptr(), M, tiled.data_ptr(), tiled_s.data_ptr(), N, K,
              fmt, None if bias is None else bias.data_ptr(), out.data_ptr(), N,
              torch.cuda.current_stream(a.device).cuda_stream)
    return out


def test_noalloc_gemm_matches_workspace_gemm(pkg, oracle_mod, dev):
    from vllm_mach_amd import _lib
    assert _lib.query("mxl_noalloc_scratch_bytes") == 32 << 20
    # c2 at M = 512 (wide kernel, three K splits: 15 MiB of partials), then smaller calls:
    # M = 128 (split), M = 16 (weight streaming, no scratch), a ragged FP6 shape
    for M, N, K, fmt in [(512, 2560, 9216, 0), (128, 2560, 9216, 0), (16, 2560, 9216, 0), (200, 1000, 768, 2)]:
        need = _lib.query("mxl_gemm_workspace_bytes_ex", M, N, K, fmt, 0, None)
        print(f"noalloc case M={M} N={N} K={K} fmt={fmt} split bytes={need}", flush=True)
        wc, ws, x, a, sa, tiled, tiled_s = _case(pkg, oracle_mod, dev, M, N, K, fmt, 11 + M)
        ref = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)  # the workspace entry point
        got = _noalloc(pkg, a, sa, tiled, tiled_s, M, N, K, fmt)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, N, K, fmt)
        assert torch.equal(_noalloc(pkg, a, sa, tiled, tiled_s, M, N, K, fmt), ref)  # repeat: same bits
        rc, rs = oracle_mod.quant_mxfp8(x, 0)
        _check(got.float().cpu().numpy(),
               oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt))))


def test_noalloc_gemm_rejects_oversized_split(pkg, dev):
    from vllm_mach_amd import _lib
    limit = _lib.query("mxl_noalloc_scratch_bytes")
    shape = None
    for M, N, K in [(512, 6144, 32768), (1024, 5120, 32768), (1024, 6144, 32768)]:
        if _lib.query("mxl_gemm_workspace_bytes_ex", M, N, K, 0, 0, None) > limit:
            shape = (M, N, K)
            break
    if shape is None:
        pytest.skip("no candidate shape splits past the scratch size")
    M, N, K = shape
    a = torch.empty((M, K), dtype=torch.uint8, device=dev)   # never read: rejected before launch
    with pytest.raises(_lib.MxlError, match="split-K scratch"):
        _lib.call("mxl_mx_gemm_noalloc", a.data_ptr(), a.data_ptr(), M, a.data_ptr(), a.data_ptr(), N, K, 0, None,
                  a.data_ptr(), N, torch.cuda.current_stream(dev).cuda_stream)
