"""The K-chunked weight-streaming GEMM (mxl_gemm_options.kernel 4, up to 128 rows):
against the oracle's dequantize-then-matmul within the GEMM bar, for every weight
format, ragged M, N and K (a short last chunk, a half last super-tile), both chunk
sizes, with a bias; and run to run bit-equal (the partials are summed in chunk order)."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import _act, _check, _weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt", [0, 2, 3])
@pytest.mark.parametrize("M", [17, 64, 100, 128])
@pytest.mark.parametrize("N,K", [(256, 2048), (200, 640), (2560, 9216), (384, 5120)])
def test_chunk_gemm_matches_oracle(pkg, oracle_mod, dev, fmt, M, N, K):
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 1100 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 1101 + M)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(3)).bfloat16().to(dev) if N == 200 else None
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    ref = oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)
    if bias is not None:
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref)) + bias.float().cpu().numpy()
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref))
    with ops.tuning(kernel=ops.KERNEL_CHUNK):
        y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, bias)
        y2 = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, bias)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    _check(y.float().cpu().numpy(), ref)


def test_chunk_gemm_plan_and_limits(pkg, dev):
    from vllm_mach_amd import _lib
    ops = pkg.ops
    opts = _lib.GemmOptions(kernel=ops.KERNEL_CHUNK)
    assert _lib.plan_name("mxl_gemm_plan_name", 128, 2560, 9216, 0, 0, options=opts) == \
        "gemm_chunk_kernel<0,4,1> + splitk_reduce8_kernel"
    assert _lib.plan_name("mxl_gemm_plan_name", 128, 2560, 2048, 2, 0, options=opts) == "gemm_chunk_kernel<2,4,1>"
    # chosen automatically where it measured fastest: K in one chunk, more n-tiles than CUs;
    # with fewer n-tiles the generic kernel measured faster
    assert _lib.plan_name("mxl_gemm_plan_name", 128, 4608, 2048, 2, 0) == "gemm_chunk_kernel<2,4,1>"
    assert _lib.plan_name("mxl_gemm_plan_name", 128, 2048, 2048, 0, 0) == "gemm_kernel<0,4,1,false,false>"
    assert _lib.plan_name("mxl_gemm_plan_name", 128, 2560, 9216, 0, 0).startswith("gemm_wide_kernel")
    with pytest.raises(_lib.MxlError):  # more than 128 rows
        _lib.plan_name("mxl_gemm_plan_name", 129, 2560, 9216, 0, 0, options=opts)
    with pytest.raises(_lib.MxlError):  # block-FP8 weights
        _lib.plan_name("mxl_gemm_plan_name", 128, 2560, 9216, 0, 1, options=opts)
