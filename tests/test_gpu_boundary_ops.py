"""GPU parity of the reference-named operators (``libmxlinear_torch.so``) and of the
``mxfp6`` package API (``vllm_mach_amd.mxfp6_api``) against the oracle, called with
the reference's own operand layouts: logical E4M3 / packed FP6 weights, swizzled
E8M0 activation and weight scales, the 64-row duplicated block-FP8 scales passed
transposed (src/vllm_mach/fp8/block_native.py:61-65), and the MoE route -> grouped
GEMM -> SwiGLU grouped GEMM -> reduce sequence of src/vllm_mach/mxfp6/moe.py:652-702.
Codes and scales must match bit for bit; GEMMs meet the north-star bar."""
import warnings

import numpy as np
import pytest
import torch

from test_gpu_gemm import _act, _check, _weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def api(pkg):
    from vllm_mach_amd import mxfp6_api
    mxfp6_api.load_library()
    return mxfp6_api


def _ref_bf16(oracle_mod, x):
    return oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(x))


@pytest.mark.parametrize("M,N,K", [(16, 2560, 4096), (64, 2560, 9216), (128, 18432, 2560), (1, 2560, 4096)])
def test_block_fp8_mm(api, oracle_mod, dev, M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    wb = (torch.randn(N, K, generator=g) * 0.02).reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    x = torch.randn(M, K, generator=g).bfloat16()
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    weight = wq.to(dev)
    sb64 = sb.repeat_interleave(2, dim=0).contiguous().to(dev)  # fp8/linear.py:137-154
    y = torch.ops.vllm_mach_block_fp8.mm(q, weight.T, s, sb64.T)
    rq, rs = oracle_mod.quant_block_fp8(x)
    ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
    _check(y.float().cpu().numpy(), ref)
    assert torch.equal(torch.ops.vllm_mach_block_fp8.mm(q, weight.T, s, sb64.T), y)  # cached tiles


@pytest.mark.parametrize("rows,transposed", [(1, True), (7, False), (64, True), (33, False)])
def test_fp8_activation_run(api, oracle_mod, dev, rows, transposed):
    H = 9216
    x = (torch.randn(rows, 2 * H, generator=torch.Generator().manual_seed(rows)) * 3).bfloat16()
    out = torch.empty((rows, H), dtype=torch.float8_e4m3fn, device=dev)
    scales = (torch.empty((H // 128, rows), dtype=torch.float32, device=dev).t() if transposed
              else torch.empty((rows, H // 128), dtype=torch.float32, device=dev))
    torch.ops.mach_fp8_activation.run(out, x.to(dev), scales, transposed)
    rq, rs = oracle_mod.silu_mul_block_fp8(x, transposed)
    assert np.array_equal(out.view(torch.uint8).cpu().numpy(), rq)
    assert np.array_equal(scales.cpu().numpy(), rs)


def test_mxfp6_quantize_and_pack_scales(api, oracle_mod, dev):
    x = _act(200, 5120, 3)
    codes, scales = torch.ops.mxfp6.quantize_mxfp8(x.to(dev))
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    assert np.array_equal(codes.cpu().numpy(), rc)
    assert np.array_equal(scales.cpu().numpy(), oracle_mod.swizzle_scales(rs, 5120))
    packed = api.pack_scales(torch.from_numpy(rs).to(dev))
    assert np.array_equal(packed.cpu().numpy(), oracle_mod.swizzle_scales(rs, 5120))
    c2, s2 = api.quantize_mxfp8_logical(x.to(dev))
    assert np.array_equal(c2.view(torch.uint8).cpu().numpy(), rc) and np.array_equal(s2.cpu().numpy(), rs)
    # [E, R, K/32]: each expert swizzled on its own
    e3 = torch.from_numpy(np.stack([rs[:100], rs[100:]])).to(dev)
    p3 = api.pack_scales(e3).cpu().numpy()
    assert np.array_equal(p3[1], oracle_mod.swizzle_scales(rs[100:], 5120))


@pytest.mark.parametrize("M,N,K,tactic,splits", [
    (16, 2560, 9216, -1, 1),     # weight streaming
    (40, 2560, 9216, -1, 1),     # generic kernel
    (128, 2560, 9216, -1, 1),    # wide kernel, split K
    (300, 2048, 2304, 1, 3),     # forced wide kernel, three K splits, ragged M
    (512, 2560, 9216, -1, 1),
])
def test_mxfp8_sm120_gemm_swizzled_scales(api, oracle_mod, dev, M, N, K, tactic, splits):
    """The reference's native GEMM call (native_backend.py:193-205): swizzled activation
    and weight scales, a workspace from allocate_workspace, a caller-given output."""
    wc, ws, _ = _weights(oracle_mod, N, K, 0, 0.02, 100 + M)
    b = torch.from_numpy(wc).to(dev).view(torch.float8_e4m3fn)
    sb = torch.from_numpy(oracle_mod.swizzle_scales(ws, K)).to(dev)
    x = _act(M, K, 50 + M)
    codes, sa = torch.ops.mxfp6.quantize_mxfp8(x.to(dev))
    a = codes.view(torch.float8_e4m3fn)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    work = torch.ops.mxfp8_sm120.allocate_workspace(a, b, sa, sb, out, tactic, splits, 1, 0)
    y = torch.ops.mxfp8_sm120.gemm(a, b, sa, sb, out, work, tactic, splits, 1, 0)
    assert y.data_ptr() == out.data_ptr()
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    _check(y.float().cpu().numpy(), _ref_bf16(oracle_mod, oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 0)))
    # the same kernel with logical scales gives the same bits
    if tactic == -1:
        tiled, tiled_s = pkg_pack(dev, wc, ws)
        y2 = torch.ops.mach_amd.mx_gemm(a, torch.from_numpy(rs).to(dev), tiled, tiled_s, N, K, 0, None)
        assert torch.equal(y, y2)
        y3 = torch.ops.mxfp8_sm120.gemm(a, b, sa, sb)  # fresh output, internal workspace
        assert torch.equal(y3, y)


def pkg_pack(dev, wc, ws):
    import __graft_entry__
    ops = __graft_entry__.load_package().ops
    return ops.pack_weight(torch.from_numpy(wc).to(dev), torch.from_numpy(ws).to(dev), 0)


def test_mxfp8_sm120_gemm_from_float_and_capture(api, oracle_mod, dev):
    M, N, K = 16, 2048, 2048
    wc, ws, _ = _weights(oracle_mod, N, K, 0, 0.02, 9)
    w = torch.from_numpy(wc).to(dev).view(torch.float8_e4m3fn)
    wsw = api.pack_scales(torch.from_numpy(ws).to(dev))
    x = _act(M, K, 4).to(dev)
    y = torch.ops.mxfp8_sm120.gemm_from_float(x, w, wsw)
    rc, rs = oracle_mod.quant_mxfp8(x.cpu(), 0)
    _check(y.float().cpu().numpy(), _ref_bf16(oracle_mod, oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 0)))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = torch.ops.mxfp8_sm120.gemm_from_float(x, w, wsw)
        for _ in range(3):
            graph.replay()
            stream.synchronize()
            assert torch.equal(out, y)
            assert torch.equal(torch.ops.mxfp8_sm120.gemm_from_float(x, w, wsw), y)
    torch.cuda.current_stream().wait_stream(stream)
    # an unprepared weight is refused during capture (the aborted capture records nothing,
    # which torch reports as an empty graph)
    w2 = w.clone()
    with torch.cuda.stream(stream), warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="The CUDA Graph is empty")
        g2 = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="before graph capture"):
            with torch.cuda.graph(g2, stream=stream):
                torch.ops.mxfp8_sm120.gemm_from_float(x, w2, wsw)
    torch.cuda.synchronize()


@pytest.mark.parametrize("M", [1, 16, 256])
def test_mxfp6_gemm_from_float_e3m2(api, oracle_mod, dev, M):
    N, K = 4352, 5120
    wc, ws, stored = _weights(oracle_mod, N, K, 3, 0.015, 70 + M)
    w = torch.from_numpy(stored).to(dev)
    wsw = api.pack_scales(torch.from_numpy(ws).to(dev))
    x = _act(M, K, 8 + M)
    y = torch.ops.mxfp6.gemm_from_float(x.to(dev), w, wsw, N, 1.0, torch.bfloat16)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    _check(y.float().cpu().numpy(), _ref_bf16(oracle_mod, oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 3)))
    # pre-quantized codes with swizzled scales (ar_norm.py:144-147)
    codes, sa = torch.ops.mxfp6.quantize_mxfp8(x.to(dev))
    y2 = torch.ops.mxfp6.gemm_w6a8_pdl(codes, w, sa, wsw, M, N, K, 1.0, torch.bfloat16)
    assert torch.equal(y2, y)
    y3 = torch.ops.mxfp6.gemm_from_float(x.to(dev), w, wsw, N, 0.5, torch.float16)
    assert y3.dtype == torch.float16
    ref16 = (oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 3) * np.float32(0.5)).astype(np.float16)
    _check(y3.float().cpu().numpy(), ref16.astype(np.float32))


def _integer_operands(oracle_mod, M, N, K, seed):
    """Integer-valued bf16 operands in [-7, 7]: every value is exact in MXFP8 (floor_carry175)
    and in E3M2 (OCP floor rule), and every fp32 partial sum of their products is an integer
    below 2^24, so any summation order gives the exact product."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(-7, 8, (N, K), generator=g).float().bfloat16()
    x = torch.randint(-7, 8, (M, K), generator=g).float().bfloat16()
    wc, ws = oracle_mod.quant_mxfp6(w, 3)
    assert np.array_equal(oracle_mod.dequant_mx(wc, ws, 3), w.float().numpy())
    xc, xs = oracle_mod.quant_mxfp8(x, 0)
    assert np.array_equal(oracle_mod.dequant_mx(xc, xs, 0), x.float().numpy())
    exact = x.double().numpy() @ w.double().numpy().T
    assert np.abs(exact).max() < 2 ** 24
    return x, oracle_mod.pack_fp6(wc), ws, exact


@pytest.mark.parametrize("M", [1, 4, 16, 256])
@pytest.mark.parametrize("dtype,alpha", [(torch.float16, 0.375), (torch.float16, 1.0), (torch.bfloat16, 0.5),
                                         (torch.bfloat16, 1.0)])
def test_mxfp6_output_rounds_once(api, oracle_mod, dev, M, dtype, alpha):
    """mxfp6::gemm_from_float / gemm_w6a8_pdl / gemm_from_swiglu with (alpha, dtype): the fp32
    sum is scaled in fp32 and rounded once to the requested dtype (src/vllm_mach/mxfp6/
    dense.py:122-129).  With exact operands the output must equal round_dtype(alpha * exact)
    bit for bit; a bf16 rounding on the way to fp16 would not (it keeps 8 of fp16's 11
    significand bits).  Covers the one-row fused launch (M = 1), the weight-streaming kernel,
    the two-call fused path (M = 4) and the wide kernel with its K split (M = 256)."""
    N, K = 1024, 5120
    x, wp, ws, exact = _integer_operands(oracle_mod, M, N, K, 40 + M)
    w = torch.from_numpy(wp).to(dev)
    wsw = api.pack_scales(torch.from_numpy(ws).to(dev))
    expected = torch.from_numpy((exact.astype(np.float32) * np.float32(alpha))).to(dtype)
    y = torch.ops.mxfp6.gemm_from_float(x.to(dev), w, wsw, N, alpha, dtype)
    assert y.dtype == dtype and torch.equal(y.cpu(), expected)
    codes, sa = torch.ops.mxfp6.quantize_mxfp8(x.to(dev))
    y2 = torch.ops.mxfp6.gemm_w6a8_pdl(codes, w, sa, wsw, M, N, K, alpha, dtype)
    assert torch.equal(y2, y)
    if dtype == torch.float16 and alpha != 1.0:  # the double rounding this replaces differs
        assert not torch.equal(y.cpu(), expected.bfloat16().to(dtype))


@pytest.mark.parametrize("M", [1, 4])
def test_mxfp6_gemm_from_swiglu_rounds_once(api, oracle_mod, dev, M):
    """gemm_from_swiglu with (alpha, fp16): one rounding of alpha times the GEMM of the
    producer's codes, for the one-row launch and the two-call path."""
    N, K = 1024, 2048
    g = torch.Generator().manual_seed(7 + M)
    wb = torch.randint(-7, 8, (N, K), generator=g).float().bfloat16()
    wc, ws = oracle_mod.quant_mxfp6(wb, 3)
    w = torch.from_numpy(oracle_mod.pack_fp6(wc)).to(dev)
    wsw = api.pack_scales(torch.from_numpy(ws).to(dev))
    gu = torch.randn(M, 2 * K, generator=g).bfloat16()
    rc, rs = oracle_mod.swiglu_mxfp8(gu, oracle_mod.RULE_CEIL_DIV448)
    y16 = torch.ops.mxfp6.gemm_from_swiglu(gu.to(dev), w, wsw, N, 0.375, torch.float16)
    ref = oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 3) * np.float32(0.375)
    _check(y16.float().cpu().numpy(), ref.astype(np.float16).astype(np.float32))
    # the same launch in bf16 without scaling: the fp16 output is the fp32 sum scaled and
    # rounded once, so it carries more of the sum than the bf16 output does
    y = torch.ops.mxfp6.gemm_from_swiglu(gu.to(dev), w, wsw, N, 1.0, torch.bfloat16)
    e16 = np.linalg.norm(y16.double().cpu().numpy() - ref) / np.linalg.norm(ref)
    e_bf = np.linalg.norm(y.double().cpu().numpy() * 0.375 - ref) / np.linalg.norm(ref)
    assert e16 < 0.25 * e_bf, (e16, e_bf)


@pytest.mark.parametrize("M", [1, 4])
def test_mxfp6_gemm_from_swiglu(api, oracle_mod, dev, M):
    N, K = 5120, 8704
    wc, ws, stored = _weights(oracle_mod, N, K, 3, 0.015, 30 + M)
    w = torch.from_numpy(stored).to(dev)
    wsw = api.pack_scales(torch.from_numpy(ws).to(dev))
    gu = torch.randn(M, 2 * K, generator=torch.Generator().manual_seed(M)).bfloat16()
    y = torch.ops.mxfp6.gemm_from_swiglu(gu.to(dev), w, wsw, N, 1.0, torch.bfloat16)
    rc, rs = oracle_mod.swiglu_mxfp8(gu, oracle_mod.RULE_CEIL_DIV448)
    _check(y.float().cpu().numpy(), _ref_bf16(oracle_mod, oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 3)))


@pytest.mark.parametrize("E,T,topk,mapped", [(8, 40, 2, False), (16, 200, 4, True)])
def test_moe_api_sequence(api, oracle_mod, dev, E, T, topk, mapped):
    """quantize -> route_mxfp8_out -> grouped_gemm_w6a8_out -> silu_and_mul_mxfp8_grouped +
    grouped_gemm_w6a8_out -> moe_reduce_out, as Mxfp6Sm120Experts.apply calls them, against
    the per-expert oracle; with an expert_map, routes of non-local experts drop out."""
    H, I = 512, 256
    g = torch.Generator().manual_seed(E + T)
    w13 = [_weights(oracle_mod, 2 * I, H, 3, 0.05, 500 + e) for e in range(E)]
    w2 = [_weights(oracle_mod, H, I, 3, 0.05, 600 + e) for e in range(E)]
    W13 = torch.from_numpy(np.stack([p[2] for p in w13])).to(dev)
    W2 = torch.from_numpy(np.stack([p[2] for p in w2])).to(dev)
    S13 = api.pack_scales(torch.from_numpy(np.stack([p[1] for p in w13])).to(dev))
    S2 = api.pack_scales(torch.from_numpy(np.stack([p[1] for p in w2])).to(dev))
    hidden = torch.randn(T, H, generator=g).bfloat16()
    logits = torch.randn(T, 2 * E if mapped else E, generator=g)
    wts, ids = torch.topk(torch.softmax(logits, -1), topk, dim=-1)
    wts = (wts / wts.sum(-1, keepdim=True)).float()
    ids = ids.int()
    expert_map = None
    local_ids = ids
    if mapped:  # global experts [0, 2E): the even ones are local (e/2), the odd ones elsewhere
        gm = torch.full((2 * E,), -1, dtype=torch.int32)
        gm[0::2] = torch.arange(E, dtype=torch.int32)
        expert_map = gm.to(dev)
        local_ids = gm[ids.long()]
    R = T * topk
    quantized, logical = api.quantize_mxfp8_logical(hidden.to(dev))
    permuted = torch.empty((R, H), dtype=torch.float8_e4m3fn, device=dev)
    packed, offsets, scale_offsets, inverse = api.route_mxfp8_out(quantized, logical, ids.to(dev), expert_map, E,
                                                                  permuted)
    gemm1 = torch.empty((R, 2 * I), dtype=torch.bfloat16, device=dev)
    api.grouped_gemm_w6a8_out(gemm1, permuted, packed, W13, S13, offsets, scale_offsets)
    act, scales, so2 = api.silu_and_mul_mxfp8_grouped(gemm1, offsets, scale_offsets)
    gemm2 = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
    api.grouped_gemm_w6a8_out(gemm2, act, scales, W2, S2, offsets, so2)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    api.moe_reduce_out(out, gemm2, wts.to(dev), inverse)
    # the same kernels as Mxfp6Experts.apply, which gathers rows instead of permuting them:
    # identical bits
    import __graft_entry__
    experts = __graft_entry__.load_package().Mxfp6Experts(fmt=3)
    e1, e2 = experts.process_weights_after_loading(
        W13, torch.from_numpy(np.stack([p[1] for p in w13])).to(dev), W2,
        torch.from_numpy(np.stack([p[1] for p in w2])).to(dev))
    out2 = torch.empty_like(out)
    experts.apply(out2, hidden.to(dev), e1, e2, wts.to(dev), ids.to(dev), "silu", 2 * E if mapped else E,
                  expert_map, None, None, None, None, None, False)
    assert torch.equal(out, out2)
    # oracle: experts restricted to the local ones (dropped routes contribute nothing); the
    # whole-layer bar of tests/native_mxfp6/test_moe.py:248 (the bf16 gate_up intermediate
    # flips a few MXFP8 codes)
    ref = oracle_mod.bf16_to_f32(oracle_mod.moe_ref(
        hidden, np.stack([p[0] for p in w13]), np.stack([p[1] for p in w13]), np.stack([p[0] for p in w2]),
        np.stack([p[1] for p in w2]), wts.numpy(), local_ids.numpy(), fmt=3))
    got = out.float().cpu().numpy()
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2
    np.testing.assert_allclose(got, ref, rtol=0.03, atol=0.03)


@pytest.mark.parametrize("M,N,K", [(32, 2048, 2560), (64, 1024, 4096), (7, 512, 1024)])
def test_dual_gemm_out(api, oracle_mod, dev, pkg, M, N, K):
    """mxfp6.mxfp8_dual.quantize + gemm_out (mxfp8/dual.py:42-45) with swizzled scales:
    bit-identical to this package's two-limb GEMM on logical scales, within the GEMM bar
    of the oracle's exact two-limb sum."""
    wc, ws, _ = _weights(oracle_mod, N, K, 0, 0.02, 41 + M)
    w = torch.from_numpy(wc).to(dev).view(torch.float8_e4m3fn)
    wsw = api.pack_scales(torch.from_numpy(ws).to(dev))
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: K // 50]] *= 30
    x = x.bfloat16()
    hi, s_hi, res, s_res = api.mxfp8_dual.quantize(x.to(dev))
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    api.mxfp8_dual.gemm_out(hi, w, s_hi, wsw.view(-1), res, s_res, out)
    ops = pkg.ops
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(wc).to(dev), torch.from_numpy(ws).to(dev), 0)
    assert torch.equal(out, ops.mx_gemm_from_float_dual(x.to(dev), tiled, tiled_s, N, 0))
    rh, rsh, rr, rsr = oracle_mod.quant_mxfp8_dual(x, 0)
    ref = oracle_mod.mx_gemm_ref(rh, rsh, wc, ws, 0) + oracle_mod.mx_gemm_ref(rr, rsr, wc, ws, 0)
    _check(out.float().cpu().numpy(), _ref_bf16(oracle_mod, ref))
    # the PDL-named entry points are the same work
    y = torch.ops.mxfp8_sm120.gemm_from_float(x.to(dev), w, wsw)
    assert torch.equal(torch.ops.mxfp8_sm120.gemm_from_float_pdl(x.to(dev), w, wsw), y)
    q, sq = torch.ops.mxfp6.quantize_mxfp8(x.to(dev))
    q2, sq2 = torch.ops.mxfp6.quantize_mxfp8_pdl(x.to(dev))
    assert torch.equal(q, q2) and torch.equal(sq, sq2)
    assert torch.equal(torch.ops.mxfp8_sm120.gemm_pdl(q.view(torch.float8_e4m3fn), w, sq, wsw), y)
    # the dense runtime module (mxfp6.mxfp8)
    assert torch.equal(api.mxfp8.gemm_from_float(x.to(dev), api.mxfp8.MXFP8Tensor(w, wsw, N, K)), y)


@pytest.mark.parametrize("M", [1, 16, 200])
def test_dense_w6a8_api(api, oracle_mod, dev, M):
    """PackedMXFP6Tensor / gemm_from_float / gemm_w6a8 / warmup_w6a8 of the mxfp6 package
    (warmup.py:55-67, sm120_owner_prefill.py:56-63, tests/native_mxfp6/test_moe.py:232)."""
    N, K = 1024, 2048
    wc, ws, stored = _weights(oracle_mod, N, K, 3, 0.015, 90 + M)
    weight = api.PackedMXFP6Tensor(torch.from_numpy(stored).to(dev), api.pack_scales(torch.from_numpy(ws).to(dev)),
                                   N, K)
    x = _act(M, K, 7 + M).to(dev)
    api.warmup_w6a8(x, weight, out_dtype=torch.bfloat16, iterations=1)
    y = api.gemm_from_float(x, weight, out_dtype=torch.bfloat16)
    rc, rs = oracle_mod.quant_mxfp8(x.cpu(), 0)
    _check(y.float().cpu().numpy(), _ref_bf16(oracle_mod, oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 3)))
    operand = api.quantize_mxfp8(x)
    assert (operand.rows, operand.k) == (M, K)
    assert torch.equal(api.gemm_w6a8(operand, weight, out_dtype=torch.bfloat16), y)
    assert api.gemm_from_float(x, weight, out_dtype=torch.float16).dtype == torch.float16
