"""One-launch producer + GEMM at decode sizes (M <= 16): the producer waves of the
weight-streaming GEMM compute the activation codes and a grid-wide handoff passes them
to the weight waves (mxl_swiglu_mx_gemm, mxl_quant_mx_gemm, mxl_block_fp8_quant_gemm).

Bar: bit-identical to the standalone producer followed by the GEMM (the same codes, the
same MFMA chain and sums), every weight format and scale rule, special values included;
the oracle's dequantize-then-matmul within the GEMM bar (relative Frobenius 1e-3, max
elementwise 1e-2 max|ref|); back-to-back launches on one stream, launches on several
streams and graph replays, so the handoff counters are seen to reset.
"""
import numpy as np
import pytest
import torch

from test_gpu_gemm import _act, _check, _weights

pytestmark = pytest.mark.gpu


def _eq(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def _swiglu_input(M, K, seed, special=True):
    g = torch.Generator().manual_seed(seed)
    gu = (torch.randn(M, 2 * K, generator=g) * 2).bfloat16()
    if special:
        gu[0, 5] = float("inf")  # an infinite amax block and a NaN lane: the special-value path
        gu[M - 1, K + 40] = float("nan")
    return gu


@pytest.mark.parametrize("fmt", [0, 2, 3])
@pytest.mark.parametrize("rule", [1, 2])
@pytest.mark.parametrize("M", [1, 2, 7, 16])
@pytest.mark.parametrize("N,K", [(160, 128), (200, 640), (2560, 9216), (96, 4608), (512, 2048)])
def test_swiglu_one_launch_bit_identical(pkg, oracle_mod, dev, fmt, rule, M, N, K):
    ops = pkg.ops
    if not ops.swiglu_row_fusable(M, K, rule, fmt):
        assert fmt != 0 and K > 7680  # FP6 past one super-tile per wave: two launches
        return
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 600 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(9)).bfloat16().to(dev) if N == 200 else None
    gu = _swiglu_input(M, K, 601 + M + K).to(dev)
    a, sa = torch.ops.mach_amd.swiglu_mxfp8(gu, rule, False)
    y_ref = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, bias)
    y = torch.ops.mach_amd.swiglu_mx_gemm(gu, tiled, tiled_s, N, fmt, rule, bias)
    assert _eq(y, y_ref)
    finite = _swiglu_input(M, K, 602 + M + K, special=False)
    y = torch.ops.mach_amd.swiglu_mx_gemm(finite.to(dev), tiled, tiled_s, N, fmt, rule, None)
    assert _eq(y, ops.swiglu_mx_down(finite.to(dev), tiled, tiled_s, N, fmt, rule))  # the layer path
    if M * N >= 2048:  # the Frobenius bar needs enough outputs for its bf16 rounding noise to average
        rc, rs = oracle_mod.swiglu_mxfp8(finite, rule)
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
        _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("fmt", [0, 2, 3])
@pytest.mark.parametrize("rule", [0, 1, 2])
@pytest.mark.parametrize("M", [1, 3, 16])
@pytest.mark.parametrize("N,K", [(160, 128), (200, 640), (2048, 2048), (17408, 5120), (2560, 9216)])
def test_quant_one_launch_bit_identical(pkg, oracle_mod, dev, fmt, rule, M, N, K):
    ops = pkg.ops
    if not ops.quant_row_fusable(M, K, rule, fmt):
        assert fmt != 0 and K > 7680
        return
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 700 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(7)).bfloat16().to(dev) if N == 200 else None
    x = _act(M, K, 701 + M + K)
    special = x.clone()
    special[0, 3] = float("inf")
    special[M - 1, 40] = float("nan")
    special[0, 70] = -float("inf")
    special[M - 1, 100] = 1e-40
    # a block below 2^-119 (rule 0's E8M0 code wraps to 255), a zero block, a negative NaN
    # and a signalling NaN: the in-register quantizer's binary32 branch and its scaled
    # conversions' block conditions
    if K >= 192:
        special[(M - 1) // 2, 128:160] = torch.linspace(-3e-37, 3e-37, 32)
        special[(M - 1) // 2, 160:192] = 0.0
    special[0, 200 % K] = torch.tensor([-64], dtype=torch.int16).view(torch.bfloat16)  # 0xFFC0
    special[M - 1, 250 % K] = torch.tensor([0x7F81], dtype=torch.int16).view(torch.bfloat16)
    inreg = ops.quant_rows_inreg(M, K, rule, fmt)
    for rows in (x, special):
        xd = rows.to(dev)
        a, sa = torch.ops.mach_amd.quantize_mxfp8(xd, rule)
        y_ref = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, bias)
        y = torch.ops.mach_amd.quant_mx_gemm(xd, tiled, tiled_s, N, fmt, rule, bias)
        assert _eq(y, y_ref)
        # each scheme by name: 0 the producer waves and handoff, 3 the GEMM's own wavefronts
        from vllm_mach_amd import _lib
        for kernel in (0, 3):
            y_k = torch.empty_like(y_ref)
            try:
                _lib.call("mxl_quant_mx_gemm_ex", xd.data_ptr(), M, K, rule, tiled.data_ptr(), tiled_s.data_ptr(),
                          N, fmt, bias.data_ptr() if bias is not None else None, y_k.data_ptr(), N,
                          _lib.options_ptr(_lib.GemmOptions(kernel=kernel)),
                          torch.cuda.current_stream(dev).cuda_stream)
            except _lib.MxlError as e:
                assert "unsupported" in str(e) and (kernel == 0 or not inreg), (kernel, str(e))
                continue
            assert kernel == 0 or inreg
            assert _eq(y_k, y_ref), kernel
    # the layer path takes one launch where the GEMM's wavefronts quantize (one row, or up
    # to 16 rows at K <= 6144), else the two launches (faster than the handoff)
    assert inreg == (M == 1 or K <= 6144)
    before = dict(ops._COUNTS)
    y_layer = ops.mx_gemm_from_float(x.to(dev), tiled, tiled_s, N, fmt, rule)
    assert ops._COUNTS.get("quant_mx_gemm", 0) == before.get("quant_mx_gemm", 0) + int(inreg)
    y = torch.ops.mach_amd.quant_mx_gemm(x.to(dev), tiled, tiled_s, N, fmt, rule, None)
    assert _eq(y, y_layer)
    if M * N >= 2048 and N * K <= 2048 * 2048:
        rc, rs = oracle_mod.quant_mxfp8(x, rule)
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
        _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("rule", [0, 1, 2])
@pytest.mark.parametrize("K", [4096, 6144])  # the wave-wide and the slice-by-slice forms
def test_quant_rows_inreg_every_value_at_every_scale(pkg, dev, rule, K):
    # the in-register quantizer against quantizer + GEMM on every (bf16 value, E8M0
    # scale) pair: an identity weight makes each output element one activation code times
    # its scale, so a code that differs shows (outputs below bf16's subnormal range
    # aside, which both paths flush alike)
    from test_gpu_quant import _every_value_at_every_scale
    ops = pkg.ops
    N = K
    x = _every_value_at_every_scale().reshape(-1)
    x = torch.cat([x, torch.zeros((-x.numel()) % (16 * K), dtype=torch.bfloat16)]).reshape(-1, K)
    assert ops.quant_rows_inreg(16, K, rule, ops.E4M3)
    eye = torch.zeros(N, K, dtype=torch.uint8)
    eye[torch.arange(N), torch.arange(K)] = 0x38  # E4M3 1.0
    tiled, tiled_s = ops.pack_weight(eye.to(dev), torch.full((N, K // 32), 127, dtype=torch.uint8, device=dev),
                                     ops.E4M3)
    xd = x.to(dev)
    for r0 in range(0, xd.shape[0], 16):
        rows = xd[r0:r0 + 16]
        a, sa = torch.ops.mach_amd.quantize_mxfp8(rows, rule)
        y_ref = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, ops.E4M3, None)
        y = torch.ops.mach_amd.quant_mx_gemm(rows, tiled, tiled_s, N, ops.E4M3, rule, None)
        assert _eq(y, y_ref), r0


@pytest.mark.parametrize("K", [640, 2176, 2560, 8192])
def test_block_fp8_row_inreg_part_supertile(pkg, dev, K):
    # one row quantized by the GEMM's wavefronts where the last super-tile is partly past K
    # (640, 2176: slices past K take the last slice's scale, as the clamped two-launch load
    # does -- an infinity in the last group makes both outputs NaN alike) and at the two
    # super-tiles per wave of K = 8192
    ops = pkg.ops
    N = 256
    wq, sb = _block_weights(N, K, 900 + K)
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    sbd = sb.to(dev)
    assert ops.block_row_inreg(1, K)
    g = torch.Generator().manual_seed(901 + K)
    for case in range(3):
        x = torch.randn(1, K, generator=g).bfloat16()
        if case == 1:
            x[0, K - 100] = float("inf")
        if case == 2:
            x[0, K - 128:] = 0.0
            x[0, 3] = float("nan")
        xd = x.to(dev)
        q, s = torch.ops.mach_amd.quantize_block_fp8(xd)
        y_ref = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sbd, N, K, None)
        y = torch.ops.mach_amd.block_fp8_quant_gemm(xd, tiled, sbd, N, None)
        assert _eq(y, y_ref), case


def _block_weights(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    wb = w.reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    return wq, sb


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("N,K", [(256, 512), (18432, 2560), (384, 6144), (256, 3584)])
def test_block_fp8_one_launch_bit_identical(pkg, oracle_mod, dev, M, N, K):
    ops = pkg.ops
    assert ops.block_row_fusable(M, K)
    wq, sb = _block_weights(N, K, 800 + K)
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    sbd = sb.to(dev)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(5)).bfloat16().to(dev) if N == 384 else None
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(801 + M)).bfloat16()
    special = x.clone()
    special[0, 7] = float("nan")
    special[M - 1, 200] = float("inf")
    special[0, 300] = 0.0
    special[M - 1, : min(K, 128)] = 0.0  # an all-zero group: the 1e-10 floor
    inreg = ops.block_row_inreg(M, K)
    assert inreg == (M == 1)
    from vllm_mach_amd import _lib
    for rows in (x, special):
        xd = rows.to(dev)
        q, s = torch.ops.mach_amd.quantize_block_fp8(xd)
        y_ref = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sbd, N, K, bias)
        y = torch.ops.mach_amd.block_fp8_quant_gemm(xd, tiled, sbd, N, bias)
        assert _eq(y, y_ref)
        # each scheme by name: 0 the producer waves and handoff, 3 the GEMM's own wavefronts
        for kernel in (0, 3):
            y_k = torch.empty_like(y_ref)
            try:
                _lib.call("mxl_block_fp8_quant_gemm_ex", xd.data_ptr(), M, K, tiled.data_ptr(), sbd.data_ptr(), N,
                          bias.data_ptr() if bias is not None else None, y_k.data_ptr(), N,
                          _lib.options_ptr(_lib.GemmOptions(kernel=kernel)), torch.cuda.current_stream(dev).cuda_stream)
            except _lib.MxlError as e:
                assert "unsupported" in str(e) and (kernel == 0 or not inreg), (kernel, str(e))
                continue
            assert kernel == 0 or inreg
            assert _eq(y_k, y_ref), kernel
    # the layer path: one launch for one row (the wavefronts' own quantization), else the
    # two launches (faster than the handoff), with the same bits
    before = dict(ops._COUNTS)
    y = ops.block_fp8_from_float(x.to(dev), tiled, sbd, N)
    assert ops._COUNTS.get("block_fp8_quant_gemm", 0) == before.get("block_fp8_quant_gemm", 0) + int(inreg)
    assert _eq(y, torch.ops.mach_amd.block_fp8_quant_gemm(x.to(dev), tiled, sbd, N, None))
    if M * N >= 2048 and N * K <= 2_500_000:
        rq, rs = oracle_mod.quant_block_fp8(x)
        ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(),
                                                                   sb.numpy()))
        _check(y.float().cpu().numpy(), ref)


def test_one_launch_back_to_back_and_streams(pkg, oracle_mod, dev):
    """Many launches in a row on one stream, with shapes changing the grid size between
    them, then on three other streams at once: every result equals its two-launch
    counterpart, so the handoff counters reset after each launch and the slots of
    different streams stay apart."""
    ops = pkg.ops
    shapes = [(2560, 9216, 16), (96, 512, 3), (2048, 2048, 16), (4096, 2048, 1), (160, 128, 8)]
    cases = []
    for i, (N, K, M) in enumerate(shapes):
        wc, ws, stored = _weights(oracle_mod, N, K, 0, 0.02, 900 + i)
        tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), 0)
        x = _act(M, K, 901 + i).to(dev)
        a, sa = torch.ops.mach_amd.quantize_mxfp8(x, 0)
        cases.append((N, K, tiled, tiled_s, x, torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, 0, None)))
    outs = []
    for rep in range(4):
        for N, K, tiled, tiled_s, x, _ in cases:
            outs.append(torch.ops.mach_amd.quant_mx_gemm(x, tiled, tiled_s, N, 0, 0, None))
    torch.cuda.synchronize()
    for i, y in enumerate(outs):
        assert _eq(y, cases[i % len(cases)][5]), i
    streams = [torch.cuda.Stream() for _ in range(3)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got = [[] for _ in streams]
    for rep in range(3):
        for si, s in enumerate(streams):
            with torch.cuda.stream(s):
                N, K, tiled, tiled_s, x, _ = cases[(si + rep) % len(cases)]
                got[si].append(torch.ops.mach_amd.quant_mx_gemm(x, tiled, tiled_s, N, 0, 0, None))
    torch.cuda.synchronize()
    for si in range(len(streams)):
        for rep, y in enumerate(got[si]):
            assert _eq(y, cases[(si + rep) % len(cases)][5]), (si, rep)


@pytest.mark.parametrize("kind", ["swiglu", "quant", "block"])
def test_one_launch_graph_replay(pkg, oracle_mod, dev, kind):
    """The one-launch op captured in a graph at 16 rows: each replay with new inputs equals
    the eager two-launch path bit for bit, with eager one-launch calls on the same stream
    between the replays."""
    ops = pkg.ops
    M = 16
    if kind == "block":
        N, K = 18432, 2560
        wq, sb = _block_weights(N, K, 950)
        w, s_w = ops.pack_weight(wq.to(dev), None, 0)[0], sb.to(dev)
        x = torch.randn(M, K, device=dev).bfloat16()

        def run():
            return torch.ops.mach_amd.block_fp8_quant_gemm(x, w, s_w, N, None)

        def eager():
            q, s = torch.ops.mach_amd.quantize_block_fp8(x)
            return torch.ops.mach_amd.block_fp8_gemm(q, s, w, s_w, N, K, None)
    else:
        N, K = (2560, 9216) if kind == "swiglu" else (17408, 5120)
        fmt = 0 if kind == "swiglu" else 2
        wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 951)
        w, s_w = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
        x = torch.randn(M, 2 * K if kind == "swiglu" else K, device=dev).bfloat16()

        def run():
            if kind == "swiglu":
                return torch.ops.mach_amd.swiglu_mx_gemm(x, w, s_w, N, fmt, 1, None)
            return torch.ops.mach_amd.quant_mx_gemm(x, w, s_w, N, fmt, 0, None)

        def eager():
            if kind == "swiglu":
                a, sa = torch.ops.mach_amd.swiglu_mxfp8(x, 1, False)
            else:
                a, sa = torch.ops.mach_amd.quantize_mxfp8(x, 0)
            return torch.ops.mach_amd.mx_gemm(a, sa, w, s_w, N, K, fmt, None)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y = run()
        gen = torch.Generator(device=dev).manual_seed(952)
        for scale in (2.0, 0.5, 0.0, 3.0):
            x.normal_(generator=gen).mul_(scale)
            graph.replay()
            between = run()  # an eager one-launch call on the same stream and slot
            stream.synchronize()
            replayed = y.clone()
            ref = eager()
            stream.synchronize()
            assert _eq(replayed, ref) and _eq(between, ref), scale
    torch.cuda.current_stream().wait_stream(stream)


def test_one_launch_limits(pkg, dev):
    ops = pkg.ops
    assert ops.quant_row_fusable(16, 2048, 0) and not ops.quant_row_fusable(17, 2048, 0)
    assert ops.swiglu_row_fusable(16, 9216, 1) and not ops.swiglu_row_fusable(16, 9216, 0)
    # K = 8192 (16 super-tiles): the two-launch GEMM's one-super-tile-per-wave variant has no
    # room for a producer wave; one row still runs by recomputation
    assert not ops.quant_row_fusable(2, 8192, 0) and ops.quant_row_fusable(1, 8192, 0)
    assert not ops.swiglu_row_fusable(2, 9216, 1, 2) and ops.swiglu_row_fusable(1, 9216, 1, 2)
    assert ops.block_row_fusable(16, 2560) and not ops.block_row_fusable(16, 4096)
    assert not ops.block_row_fusable(17, 2560)
    w = torch.zeros(16 * 512, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        torch.ops.mach_amd.quant_mx_gemm(torch.zeros(17, 512, dtype=torch.bfloat16, device=dev), w, w, 16, 0)
    with pytest.raises(ValueError):
        torch.ops.mach_amd.block_fp8_quant_gemm(torch.zeros(2, 4096, dtype=torch.bfloat16, device=dev), w,
                                                torch.zeros(1, 32, device=dev), 16)
