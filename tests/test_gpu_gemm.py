"""GPU parity of the block-scaled GEMMs against the oracle's dequantize-then-matmul.

Bar: relative Frobenius error <= 1e-3 and max elementwise
error <= 1e-2 * max|ref| against the fp32-accumulated reference.  Activations are
quantized on the GPU and checked bit-exact first, so the GEMM comparison isolates
the contraction.  Full-size configurations (c1..c4 shapes) run through the same
checks with the reference computed by torch (fp32 dequant + matmul on the GPU).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REL_FRO, MAX_ELEM = 1e-3, 1e-2


def _check(got: np.ndarray, ref: np.ndarray):
    err = got.astype(np.float64) - ref.astype(np.float64)
    scale = max(np.linalg.norm(ref), 1e-30)
    rel = np.linalg.norm(err) / scale
    mx = np.abs(err).max() / max(np.abs(ref).max(), 1e-30)
    assert rel <= REL_FRO and mx <= MAX_ELEM, (rel, mx)
    return rel, mx


def _act(M, K, seed, magnitude=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g) * magnitude
    x[:, torch.randperm(K, generator=g)[: max(1, K // 100)]] *= 20
    return x.bfloat16()


def _weights(oracle_mod, N, K, fmt, std, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * std).bfloat16()
    if fmt == 0:
        codes, scales = oracle_mod.quant_mxfp8(w, 0)
        stored = codes
    else:
        codes, scales = oracle_mod.quant_mxfp6(w, fmt)
        stored = oracle_mod.pack_fp6(codes)
    return codes, scales, stored


@pytest.mark.parametrize("fmt", [0, 2, 3])
@pytest.mark.parametrize("M", [1, 5, 16, 33, 64, 130])
@pytest.mark.parametrize("N,K", [(256, 512), (384, 2560), (2048, 2048)])
def test_mx_gemm_matches_oracle(pkg, oracle_mod, dev, fmt, M, N, K):
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 17 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 29 + M)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    assert np.array_equal(a.view(torch.uint8).cpu().numpy(), rc)
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    ref = oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)
    ref_bf = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref))
    _check(y.float().cpu().numpy(), ref_bf)


@pytest.mark.parametrize("M,N,K,fmt", [(9, 200, 384, 0), (100, 200, 384, 0), (100, 200, 384, 2), (257, 136, 1152, 3)])
def test_mx_gemm_bias_and_ragged_shapes(pkg, oracle_mod, dev, M, N, K, fmt):
    """K % 512 != 0 (a partial last super-tile), N not a multiple of the tile width, and a
    bf16 bias added after rounding, on both the decode and the LDS-staged kernels."""
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.05, 3)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 4)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(1)).bfloat16()
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, bias.to(dev))
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    ref = torch.from_numpy(oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt))))
    ref = (ref.bfloat16() + bias).float().numpy()
    _check(y.float().cpu().numpy(), ref)


def test_mx_gemm_zero_and_empty(pkg, dev):
    ops = pkg.ops
    N, K = 128, 256
    codes = torch.zeros(N, K, dtype=torch.uint8, device=dev)
    scales = torch.full((N, K // 32), 127, dtype=torch.uint8, device=dev)
    tiled, tiled_s = ops.pack_weight(codes, scales, 0)
    x = torch.zeros(3, K, dtype=torch.bfloat16, device=dev)
    y = ops.mx_gemm_from_float(x, tiled, tiled_s, N, 0)
    assert torch.count_nonzero(y) == 0
    e = ops.mx_gemm_from_float(x[:0], tiled, tiled_s, N, 0)
    assert tuple(e.shape) == (0, N)


def _torch_dequant(codes_u8: torch.Tensor, scales_u8: torch.Tensor, fmt: int, oracle_mod) -> torch.Tensor:
    if fmt == 0:
        v = codes_u8.view(torch.float8_e4m3fn).float()
    else:
        lut = torch.from_numpy(oracle_mod.fp6_to_f32(np.arange(64, dtype=np.uint8), fmt)).to(codes_u8.device)
        v = lut[codes_u8.long()]
    return v * torch.exp2(scales_u8.float() - 127).repeat_interleave(32, dim=1)


@pytest.mark.parametrize("name,M,N,K,fmt,std", [
    ("c1", 16, 2048, 2048, 0, 0.02),
    ("c2", 1, 2560, 9216, 0, 0.02),
    ("c2", 16, 2560, 9216, 0, 0.02),
    ("c2", 128, 2560, 9216, 0, 0.02),
    ("c2", 512, 2560, 9216, 0, 0.02),
    ("c4", 1, 17408, 5120, 2, 0.015),
    ("c4", 16, 17408, 5120, 2, 0.015),
    ("c4", 128, 17408, 5120, 2, 0.015),
    ("c4", 256, 17408, 5120, 2, 0.015),
])
def test_full_size_configs(pkg, oracle_mod, dev, name, M, N, K, fmt, std):
    """BASELINE shapes: GPU GEMM vs a torch fp32 dequant-matmul of the same codes."""
    ops = pkg.ops
    g = torch.Generator(device=dev).manual_seed(7)
    w = (torch.randn(N, K, generator=g, device=dev) * std).bfloat16()
    if fmt == 0:
        wc, ws = torch.ops.mach_amd.quantize_mxfp8(w, 0)
        wc = wc.view(torch.uint8)
        stored = wc
    else:
        c, s = oracle_mod.quant_mxfp6(w.cpu(), fmt)
        wc, ws = torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev)
        stored = torch.from_numpy(oracle_mod.pack_fp6(c)).to(dev)
    tiled, tiled_s = ops.pack_weight(stored, ws, fmt)
    x = (torch.randn(M, K, generator=g, device=dev)).bfloat16()
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x, 0)
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    ref = (_torch_dequant(a.view(torch.uint8), sa, 0, oracle_mod) @ _torch_dequant(wc, ws, fmt, oracle_mod).T)
    ref = ref.bfloat16().float()
    _check(y.float().cpu().numpy(), ref.cpu().numpy())
    del w, tiled, tiled_s
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M", [1, 3, 16, 64, 130, 512])
@pytest.mark.parametrize("N,K", [(256, 512), (18432, 2560), (2560, 9216)])
def test_block_fp8_gemm_matches_oracle(pkg, oracle_mod, dev, M, N, K):
    """Block-FP8 GEMM against the oracle's blocked product; at the full c2/c3 sizes past 64
    rows (where the C oracle's product would take minutes) against a plain torch fp32
    dequantize-then-matmul on the GPU instead, the quantized codes still checked bit for
    bit against the oracle's quantizer."""
    big = N * K > 10_000_000 and M > 64
    ops = pkg.ops
    g = torch.Generator().manual_seed(173 + M + K)
    w = (torch.randn(N, K, generator=g) * 0.02)
    wb = w.reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    x = torch.randn(M, K, generator=g).bfloat16()
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    y = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    rq, rs = oracle_mod.quant_block_fp8(x)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), rq)
    if big:
        G = K // 128
        # the codes (checked above) times their fp32 scales, in fp32: activations [M, K]
        # with one scale per 128 columns of a row, weights [N, K] with one per 128 x 128 block
        a_f = (torch.from_numpy(rq).to(dev).view(torch.float8_e4m3fn).float().view(M, G, 128)
               * torch.from_numpy(np.ascontiguousarray(rs)).to(dev).float().view(M, G, 1)).view(M, K)
        w_f = (wq.to(dev).float().view(N // 128, 128, G, 128) * sb.to(dev)[:, None, :, None]).view(N, K)
        ref = (a_f @ w_f.T).bfloat16().float().cpu().numpy()
        del a_f, w_f
        _check(y.float().cpu().numpy(), ref)
        return
    ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
    _check(y.float().cpu().numpy(), ref)


def test_graph_replay_with_changing_inputs(pkg, oracle_mod, dev):
    """Capture one MXFP8 linear call, replay with new inputs (x.normal_(), zero), as
    tests/native_mxfp6/test_mxfp8_sm120.py:40-58 does."""
    ops = pkg.ops
    M, N, K = 16, 512, 1024
    wc, ws, stored = _weights(oracle_mod, N, K, 0, 0.02, 5)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), 0)
    x = torch.randn(M, K, device=dev).bfloat16()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        ops.mx_gemm_from_float(x, tiled, tiled_s, N, 0)  # warm the per-stream workspace
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y = ops.mx_gemm_from_float(x, tiled, tiled_s, N, 0)
        for zero in (False, False, True):
            x.zero_() if zero else x.normal_()
            graph.replay()
            stream.synchronize()
            rc, rs = oracle_mod.quant_mxfp8(x.cpu(), 0)
            ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws)))
            got = y.float().cpu().numpy()
            if zero:
                assert not got.any()
            else:
                _check(got, ref)
    torch.cuda.current_stream().wait_stream(stream)


@pytest.mark.parametrize("rule", [1, 2])
@pytest.mark.parametrize("M", [1, 16, 200])
def test_swiglu_mx_down_matches_oracle(pkg, oracle_mod, dev, rule, M):
    """SwiGLU -> MXFP8 -> down projection (mach_swiglu_mxfp8_down, mxfp6/mxfp8_mlp.py:15-22;
    rule 2: the champion producer of mxfp8/swiglu_quant.py feeding the same GEMM)."""
    ops = pkg.ops
    N, K = 512, 2048
    wc, ws, stored = _weights(oracle_mod, N, K, 0, 0.02, 91)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), 0)
    gu = (torch.randn(M, 2 * K, generator=torch.Generator().manual_seed(92 + M)) * 2).bfloat16()
    y = ops.swiglu_mx_down(gu.to(dev), tiled, tiled_s, N, 0, rule)
    rc, rs = oracle_mod.swiglu_mxfp8(gu, rule)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 0)))
    _check(y.float().cpu().numpy(), ref)
    # the producer's own codes are the oracle's
    a, sa = torch.ops.mach_amd.swiglu_mxfp8(gu.to(dev), rule, False)
    assert np.array_equal(a.view(torch.uint8).cpu().numpy(), rc) and np.array_equal(sa.cpu().numpy(), rs)


@pytest.mark.parametrize("fmt", [0, 2, 3])
@pytest.mark.parametrize("rule", [1, 2])
@pytest.mark.parametrize("N,K", [(160, 128), (200, 640), (2560, 9216), (96, 12288), (512, 2048)])
def test_swiglu_row_fused_is_bit_identical(pkg, oracle_mod, dev, fmt, rule, N, K):
    """One launch (SwiGLU codes computed inside the weight-streaming GEMM) equals the
    producer followed by the GEMM bit for bit, and the oracle within the GEMM bar."""
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 300 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    g = torch.Generator().manual_seed(301 + K)
    gu = (torch.randn(1, 2 * K, generator=g) * 2).bfloat16()
    gu[0, 5] = float("inf")  # an infinite amax block and a NaN lane exercise the special-value path
    gu[0, K + 40] = float("nan")
    bias = torch.randn(N, generator=g).bfloat16().to(dev) if N == 200 else None
    gud = gu.to(dev)
    a, sa = torch.ops.mach_amd.swiglu_mxfp8(gud, rule, False)
    y_ref = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, bias)
    y = torch.ops.mach_amd.swiglu_mx_gemm(gud, tiled, tiled_s, N, fmt, rule, bias)
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    finite = (torch.randn(1, 2 * K, generator=g) * 2).bfloat16()
    y = ops.swiglu_mx_down(finite.to(dev), tiled, tiled_s, N, fmt, rule)
    rc, rs = oracle_mod.swiglu_mxfp8(finite, rule)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
    _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("fmt", [0, 2, 3])
@pytest.mark.parametrize("rule", [0, 1, 2])
@pytest.mark.parametrize("N,K", [(160, 128), (200, 640), (2560, 9216), (96, 12288), (17408, 5120)])
def test_quant_row_fused_is_bit_identical(pkg, oracle_mod, dev, fmt, rule, N, K):
    """One bf16 row quantized inside the weight-streaming GEMM (one launch) equals the
    quantizer followed by the GEMM bit for bit -- infinite, NaN and subnormal inputs and
    outlier channels included -- and the oracle within the GEMM bar."""
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 500 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(1, K, 501 + K)
    special = x.clone()
    special[0, 3] = float("inf")
    special[0, 40] = float("nan")
    special[0, 70] = -float("inf")
    special[0, 100] = 1e-40
    bias = torch.randn(N, generator=torch.Generator().manual_seed(7)).bfloat16().to(dev) if N == 200 else None
    for row in (x, special):
        xd = row.to(dev)
        a, sa = torch.ops.mach_amd.quantize_mxfp8(xd, rule)
        y_ref = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, bias)
        y = torch.ops.mach_amd.quant_mx_gemm(xd, tiled, tiled_s, N, fmt, rule, bias)
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    # mx_gemm_from_float takes the one-launch path for one row
    before = dict(ops._COUNTS)
    y = ops.mx_gemm_from_float(x.to(dev), tiled, tiled_s, N, fmt, rule)
    assert ops._COUNTS.get("quant_mx_gemm", 0) == before.get("quant_mx_gemm", 0) + 1
    if N >= 160:  # the Frobenius bar needs more than a few dozen outputs to be meaningful
        rc, rs = oracle_mod.quant_mxfp8(x, rule)
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
        _check(y.float().cpu().numpy(), ref)


def test_quant_row_fused_graph_replay_and_limits(pkg, oracle_mod, dev):
    """The one-launch quantized row under graph capture (each replay with a new row equals
    the eager call), and the shapes it refuses."""
    ops = pkg.ops
    N, K = 17408, 5120  # the W6A8 decode shape
    wc, ws, stored = _weights(oracle_mod, N, K, 2, 0.02, 77)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), 2)
    x = torch.randn(1, K, device=dev).bfloat16()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        ops.mx_gemm_from_float(x, tiled, tiled_s, N, 2)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y = ops.mx_gemm_from_float(x, tiled, tiled_s, N, 2)
        gen = torch.Generator(device=dev).manual_seed(78)
        for scale in (3.0, 0.25):
            x.normal_(generator=gen).mul_(scale)
            graph.replay()
            stream.synchronize()
            replayed = y.clone()
            a, sa = torch.ops.mach_amd.quantize_mxfp8(x, 0)
            eager = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, 2, None)
            stream.synchronize()
            assert torch.equal(replayed.view(torch.int16), eager.view(torch.int16))
    torch.cuda.current_stream().wait_stream(stream)
    assert not ops.quant_row_fusable(17, K, 0) and not ops.quant_row_fusable(1, 12416, 0)
    with pytest.raises(ValueError):
        torch.ops.mach_amd.quant_mx_gemm(torch.zeros(17, K, dtype=torch.bfloat16, device=dev), tiled, tiled_s, N, 2)


@pytest.mark.parametrize("fmt", [0, 2])
def test_swiglu_row_fused_graph_replay(pkg, oracle_mod, dev, fmt):
    """The one-launch SwiGLU down projection captured in a graph: each replay with a new
    gate/up row equals the eager call bit for bit and the oracle within the GEMM bar."""
    ops = pkg.ops
    N, K = 2560, 9216  # the decode MLP down projection of the reference's dense model
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 410 + fmt)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    gu = torch.randn(1, 2 * K, device=dev).bfloat16()
    assert ops.swiglu_row_fusable(1, K, 2)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        ops.swiglu_mx_down(gu, tiled, tiled_s, N, fmt, 2)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y = ops.swiglu_mx_down(gu, tiled, tiled_s, N, fmt, 2)
        gen = torch.Generator(device=dev).manual_seed(411)
        for scale in (2.0, 0.5, 0.0):
            gu.normal_(generator=gen).mul_(scale)
            graph.replay()
            stream.synchronize()
            replayed = y.clone()
            eager = ops.swiglu_mx_down(gu, tiled, tiled_s, N, fmt, 2)
            stream.synchronize()
            assert torch.equal(replayed.view(torch.int16), eager.view(torch.int16))
            if scale == 0.0:
                assert not replayed.float().any()
                continue
            rc, rs = oracle_mod.swiglu_mxfp8(gu.cpu(), 2)
            ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
            _check(replayed.float().cpu().numpy(), ref)
    torch.cuda.current_stream().wait_stream(stream)


def test_swiglu_row_fused_rejects_other_shapes(pkg, dev):
    ops = pkg.ops
    w = torch.zeros(16 * 512, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        torch.ops.mach_amd.swiglu_mx_gemm(torch.zeros(17, 1024, dtype=torch.bfloat16, device=dev), w, w, 16, 0, 1)
    with pytest.raises(ValueError):
        torch.ops.mach_amd.swiglu_mx_gemm(torch.zeros(1, 1024, dtype=torch.bfloat16, device=dev), w, w, 16, 0, 0)
    assert not ops.swiglu_row_fusable(1, 12800, 1) and ops.swiglu_row_fusable(1, 9216, 2)
