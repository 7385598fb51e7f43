"""GPU parity of the MoE path: token sort bit-exact, combine bit-exact, and the whole
routed-expert layer against the oracle's per-expert dense reference
(tests/native_mxfp6/test_moe.py:165-248: seed 12035, e=4, h=256, i=128, m=7, topk=2)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib_options(**kw):
    from vllm_mach_amd import _lib
    return _lib.GemmOptions(**kw)


@pytest.mark.parametrize("T,topk,E", [(7, 2, 4), (1, 8, 256), (128, 8, 256), (2048, 8, 256), (3000, 4, 64),
                                     (1, 1, 1), (100, 4, 1024), (129, 8, 256),  # one-chunk and two-chunk edges
                                     (4096, 8, 512), (300, 8, 2048)])  # histograms past LDS: three launches
def test_route_bit_exact(pkg, oracle_mod, dev, T, topk, E):
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g)
    ids = torch.topk(torch.softmax(logits, -1), topk, -1).indices.int()
    s, o, inv = torch.ops.mach_amd.moe_route(ids.to(dev), E)
    rs, ro, rinv = oracle_mod.moe_route(ids.numpy(), E)
    assert np.array_equal(o.cpu().numpy(), ro)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(inv.cpu().numpy(), rinv)


def test_route_drops_out_of_range_ids(pkg, oracle_mod, dev):
    ids = torch.tensor([[0, 5], [-1, 1], [1, 0]], dtype=torch.int32)
    s, o, inv = torch.ops.mach_amd.moe_route(ids.to(dev), 2)
    rs, ro, rinv = oracle_mod.moe_route(ids.numpy(), 2)
    n = int(ro[-1])
    assert np.array_equal(o.cpu().numpy(), ro) and np.array_equal(inv.cpu().numpy(), rinv)
    assert np.array_equal(s.cpu().numpy()[:n], rs[:n])


@pytest.mark.parametrize("T,topk,H", [(7, 2, 256), (2048, 8, 2048), (33, 1, 128), (5, 10, 512)])
def test_reduce_bit_exact(pkg, oracle_mod, dev, T, topk, H):
    g = torch.Generator().manual_seed(12035)
    y = torch.randn(T * topk, H, generator=g).bfloat16()
    w = torch.rand(T, topk, generator=g)
    w /= w.sum(-1, keepdim=True)
    inverse = torch.randperm(T * topk, generator=g).int()
    inverse[0] = -1  # a dropped route
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    torch.ops.mach_amd.moe_reduce(out, y.to(dev), w.to(dev), inverse.to(dev))
    ref = oracle_mod.moe_reduce(oracle_mod.bf16_bits(y), w.numpy(), inverse.numpy())
    assert np.array_equal(oracle_mod.bf16_bits(out), ref)


def _moe_case(oracle_mod, E, H, I, T, topk, seed, fmt=2, std=0.1):
    g = torch.Generator().manual_seed(seed)
    w13 = (torch.randn(E, 2 * I, H, generator=g) * std).bfloat16()
    w2 = (torch.randn(E, H, I, generator=g) * std).bfloat16()
    q13 = [oracle_mod.quant_mxfp6(w13[e], fmt) for e in range(E)]
    q2 = [oracle_mod.quant_mxfp6(w2[e], fmt) for e in range(E)]
    c13 = np.stack([c for c, _ in q13]); s13 = np.stack([s for _, s in q13])
    c2 = np.stack([c for c, _ in q2]); s2 = np.stack([s for _, s in q2])
    x = torch.randn(T, H, generator=g).bfloat16()
    logits = torch.randn(T, E, generator=g)
    wts, ids = torch.topk(torch.softmax(logits, -1), topk, -1)
    wts = (wts / wts.sum(-1, keepdim=True)).float()
    return c13, s13, c2, s2, x, wts, ids.int()


def _check_gemm(got, ref):
    err = got.astype(np.float64) - ref
    rel = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    mx = np.abs(err).max() / max(np.abs(ref).max(), 1e-30)
    assert rel <= 1e-3 and mx <= 1e-2, (rel, mx)


@pytest.mark.parametrize("E,H,I,T,topk,fmt", [
    (4, 256, 128, 7, 2, 2),
    (4, 256, 128, 7, 2, 3),
    (32, 2048, 512, 128, 8, 2),
    (16, 2048, 512, 512, 8, 3),
    (256, 2048, 512, 128, 8, 2),   # c5 at T = 128: every expert checked
    (256, 2048, 512, 2048, 8, 2),  # c5 at T = 2048: the default schedules (grouped wide w13,
                                   # 96-row w2 units), every expert checked
])
def test_moe_layer_matches_oracle(pkg, oracle_mod, dev, E, H, I, T, topk, fmt):
    """Each stage against the oracle on the GPU's own inputs to that stage (quantizers and
    routing bit-exact, grouped GEMMs to the GEMM bar), then the whole layer."""
    c13, s13, c2, s2, x, wts, ids = _moe_case(oracle_mod, E, H, I, T, topk, 12035, fmt)
    experts = pkg.Mxfp6Experts(fmt=fmt)
    w1, w2 = experts.process_weights_after_loading(
        torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev), torch.from_numpy(s13).to(dev),
        torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev), torch.from_numpy(s2).to(dev))
    xd, wd, idd = x.to(dev), wts.to(dev), ids.to(dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    experts.apply(out, xd, w1, w2, wd, idd, "silu", E, None, None, None, None, None, None, False)

    # stage by stage, each fed with the GPU's own output of the previous stage
    a, sa = torch.ops.mach_amd.quantize_mxfp8(xd, 0)
    ac, as_ = oracle_mod.quant_mxfp8(x, 0)
    assert np.array_equal(a.view(torch.uint8).cpu().numpy(), ac)
    sr, off, inv = torch.ops.mach_amd.moe_route(idd, E)
    rs, ro, rinv = oracle_mod.moe_route(ids.numpy(), E)
    assert np.array_equal(sr.cpu().numpy(), rs) and np.array_equal(off.cpu().numpy(), ro)
    gu = torch.ops.mach_amd.grouped_gemm(a, sa, sr, topk, off, T * topk, w1, experts.w1_scale, 2 * I, H, fmt)
    a2, sa2 = torch.ops.mach_amd.swiglu_mxfp8(gu, 1, False)
    y = torch.ops.mach_amd.grouped_gemm(a2, sa2, None, 1, off, T * topk, w2, experts.w2_scale, H, I, fmt)
    gu_h, a2_h, sa2_h, y_h = (gu.float().cpu().numpy(), a2.view(torch.uint8).cpu().numpy(),
                              sa2.cpu().numpy(), y.float().cpu().numpy())
    mc, ms = oracle_mod.swiglu_mxfp8(oracle_mod.bf16_bits(gu.cpu()), 1)
    assert np.array_equal(a2_h, mc) and np.array_equal(sa2_h, ms)
    for e in range(E):
        lo, hi = int(ro[e]), int(ro[e + 1])
        if lo == hi:
            continue
        toks = rs[lo:hi] // topk
        ref1 = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(
            oracle_mod.mx_gemm_ref(ac[toks], as_[toks], c13[e], s13[e], fmt)))
        _check_gemm(gu_h[lo:hi], ref1)
        ref2 = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(
            oracle_mod.mx_gemm_ref(a2_h[lo:hi], sa2_h[lo:hi], c2[e], s2[e], fmt)))
        _check_gemm(y_h[lo:hi], ref2)
    red = oracle_mod.moe_reduce(oracle_mod.bf16_bits(y.cpu()), wts.numpy(), rinv)
    assert np.array_equal(oracle_mod.bf16_bits(out), red)

    # whole layer against the per-expert dense reference: bf16 rounding of the gate_up
    # intermediate flips a few MXFP8 codes, so the bar is the reference's relative one
    ref = oracle_mod.bf16_to_f32(oracle_mod.moe_ref(x, c13, s13, c2, s2, wts.numpy(), ids.numpy(), fmt))
    got = out.float().cpu().numpy()
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 1e-2, rel
    if H <= 256:
        np.testing.assert_allclose(got, ref, rtol=0.03, atol=0.03)  # tests/native_mxfp6/test_moe.py:248


@pytest.mark.parametrize("E,H,I,T", [
    (4, 256, 128, 7),      # the reference's case
    (16, 512, 256, 700),   # about 88 routes per expert: both GEMMs on 96-row streaming units,
                           # routing over six token chunks in one count-and-scan launch
    (8, 1024, 512, 256),   # gate_up (K = 1024) on the wide grouped kernel: 64 rows per expert
                           # under the rotated ids (the 64-row path), mixed sizes at first
])
def test_moe_graph_replay_changing_routes(pkg, oracle_mod, dev, E, H, I, T):
    """Captured layer replayed with new hidden states and rotated expert ids
    (tests/native_mxfp6/test_moe.py:216-248)."""
    topk = 2
    c13, s13, c2, s2, x, wts, ids = _moe_case(oracle_mod, E, H, I, T, topk, 12035)
    experts = pkg.Mxfp6Experts(fmt=2)
    w1, w2 = experts.process_weights_after_loading(
        torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev), torch.from_numpy(s13).to(dev),
        torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev), torch.from_numpy(s2).to(dev))
    xd, wd, idd = x.to(dev), wts.to(dev), ids.to(dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)

    def run():
        experts.apply(out, xd, w1, w2, wd, idd, "silu", E, None, None, None, None, None, None, False)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            run()
        gen = torch.Generator(device=dev).manual_seed(77)
        for shift in range(3):
            xd.normal_(generator=gen)
            idd.copy_(torch.tensor([[(j + shift) % E, (j + shift + 1) % E] for j in range(T)], dtype=torch.int32))
            graph.replay()
            stream.synchronize()
            replayed = out.clone()
            run()  # eager on the same inputs: the replay must match it bit for bit
            stream.synchronize()
            assert torch.equal(replayed, out)
            # against the oracle: the bf16 gate_up intermediate may flip an MXFP8 code of
            # the SwiGLU output, so the whole-layer bar is the relative one
            ref = oracle_mod.bf16_to_f32(oracle_mod.moe_ref(xd.cpu(), c13, s13, c2, s2, wd.cpu().numpy(),
                                                            idd.cpu().numpy(), 2))
            got = replayed.float().cpu().numpy()
            assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2
    torch.cuda.current_stream().wait_stream(stream)


@pytest.mark.parametrize("E,N,K,T,topk,gathered,fmt,skew", [
    (256, 1024, 2048, 128, 8, True, 2, False),   # the MoE gate_up at T = 128 (c5)
    (256, 2048, 512, 128, 8, False, 2, False),   # the MoE down projection at T = 128 (c5)
    (8, 384, 1024, 20, 2, True, 0, True),        # E4M3: an expert with 30 rows (two units), empty experts
    (16, 200, 1280, 40, 2, True, 3, True),       # ragged N, K % 512 != 0 (three K waves, five n-lanes)
    (4, 256, 4096, 9, 2, True, 0, False),        # eight K waves (E4M3's largest K)
])
def test_grouped_stream_small_batch(pkg, oracle_mod, dev, monkeypatch, E, N, K, T, topk, gathered, fmt, skew):
    """Few routed rows per expert: persistent workgroups stream each expert's weights past its
    16-row tiles.  Checked against the oracle, and bit for bit against the per-expert kernel
    when both sum one super-tile per wave in K order (K <= 2048)."""
    from test_gpu_gemm import _act, _check, _weights
    ops = pkg.ops
    g = torch.Generator().manual_seed(E + N + K)
    ids = torch.randint(0, E, (T, topk), generator=g, dtype=torch.int32)
    if skew:
        ids[:15, 0] = 0
        ids[ids == 1] = 2
    parts = [_weights(oracle_mod, N, K, fmt, 0.02, 200 + e) for e in range(E)]
    w_t, s_t = ops.pack_weight(torch.from_numpy(np.stack([p_[2] for p_ in parts])).to(dev),
                               torch.from_numpy(np.stack([p_[1] for p_ in parts])).to(dev), fmt)
    routes, offsets, _ = torch.ops.mach_amd.moe_route(ids.to(dev), E)
    R = T * topk
    assert R < 32 * E  # the small-batch path
    x = _act(T if gathered else R, K, 5)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    args = (a, sa, routes, topk) if gathered else (a, sa, None, 1)
    y = torch.ops.mach_amd.grouped_gemm(*args, offsets, R, w_t, s_t, N, K, fmt)
    monkeypatch.setattr(ops, "_tuning", _lib_options(kernel=ops.KERNEL_GENERIC))
    y_ref_kernel = torch.ops.mach_amd.grouped_gemm(*args, offsets, R, w_t, s_t, N, K, fmt)
    if K <= 2048:
        assert torch.equal(y, y_ref_kernel)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    off, rt, got = offsets.cpu().numpy(), routes.cpu().numpy(), y.float().cpu().numpy()
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if lo == hi or (E > 16 and e % 8):
            continue
        rows = rt[lo:hi] // topk if gathered else np.arange(lo, hi)
        ref = oracle_mod.mx_gemm_ref(rc[rows], rs[rows], parts[e][0], parts[e][1], fmt)
        _check(got[lo:hi], oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref)))


@pytest.mark.parametrize("E,N,K,T,topk,gathered,fmt,skew", [
    (256, 2048, 512, 2048, 8, False, 2, False),  # the MoE down projection at T = 2048 (c5): the default
    (256, 1024, 2048, 2048, 8, True, 2, False),  # the MoE gate_up at T = 2048 (c5): forced, four K waves
    (8, 384, 512, 200, 2, True, 0, True),        # E4M3: an expert with > 96 rows (two units), empty experts
    (8, 200, 512, 200, 2, True, 2, True),        # 13 n-tiles over four wave lanes: each unit's partial
                                                 # round lands at its own rotated position
    (16, 200, 1280, 400, 2, True, 3, True),      # forced: ragged N, K % 512 != 0 (three K waves)
])
def test_grouped_stream_96_row_units(pkg, oracle_mod, dev, monkeypatch, E, N, K, T, topk, gathered, fmt, skew):
    """Tens of routed rows per expert: the streaming kernel over 96-row units (six m-tiles,
    each expert's weights read about once; the default where K is one super-tile) is
    bit-identical to the 16-row-unit variant -- every m-tile runs the same MFMA chain --
    and within the GEMM bar of the default schedule, the wide kernel and the oracle."""
    from test_gpu_gemm import _act, _check, _weights
    ops = pkg.ops
    g = torch.Generator().manual_seed(E + N + K + 1)
    ids = torch.randint(0, E, (T, topk), generator=g, dtype=torch.int32)
    if skew:
        ids[: T // 2, 0] = 0
        ids[ids == 1] = 2
    parts = [_weights(oracle_mod, N, K, fmt, 0.02, 400 + e) for e in range(E)]
    w_t, s_t = ops.pack_weight(torch.from_numpy(np.stack([p_[2] for p_ in parts])).to(dev),
                               torch.from_numpy(np.stack([p_[1] for p_ in parts])).to(dev), fmt)
    routes, offsets, _ = torch.ops.mach_amd.moe_route(ids.to(dev), E)
    R = T * topk
    assert 32 * E <= R <= 96 * E  # the many-row-unit path by default (K <= 512)
    x = _act(T if gathered else R, K, 6)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    args = (a, sa, routes, topk) if gathered else (a, sa, None, 1)
    y_default = torch.ops.mach_amd.grouped_gemm(*args, offsets, R, w_t, s_t, N, K, fmt)
    monkeypatch.setattr(ops, "_tuning", _lib_options(kernel=ops.KERNEL_STREAM_WIDE))
    y = torch.ops.mach_amd.grouped_gemm(*args, offsets, R, w_t, s_t, N, K, fmt)
    monkeypatch.setattr(ops, "_tuning", _lib_options(kernel=ops.KERNEL_STREAM))
    assert torch.equal(y, torch.ops.mach_amd.grouped_gemm(*args, offsets, R, w_t, s_t, N, K, fmt))
    if K <= 512:
        assert torch.equal(y, y_default)
    monkeypatch.setattr(ops, "_tuning", _lib_options(kernel=ops.KERNEL_WIDE))
    y_wide = torch.ops.mach_amd.grouped_gemm(*args, offsets, R, w_t, s_t, N, K, fmt)
    _check(y.float().cpu().numpy(), y_wide.float().cpu().numpy())
    _check(y_default.float().cpu().numpy(), y.float().cpu().numpy())
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    off, rt, got = offsets.cpu().numpy(), routes.cpu().numpy(), y.float().cpu().numpy()
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if lo == hi or (E > 16 and e % 16):
            continue
        rows = rt[lo:hi] // topk if gathered else np.arange(lo, hi)
        ref = oracle_mod.mx_gemm_ref(rc[rows], rs[rows], parts[e][0], parts[e][1], fmt)
        _check(got[lo:hi], oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref)))


@pytest.mark.parametrize("E,H,I,T,topk,fmt,mapped", [
    (4, 256, 128, 7, 2, 2, False),
    (256, 2048, 512, 128, 8, 2, False),    # c5, T = 128: both GEMMs fused (16-row units)
    (256, 2048, 512, 2048, 8, 2, False),   # c5, T = 2048: 64 rows per expert, separate producers
    (16, 512, 256, 100, 4, 3, True),       # E3M2 experts, an expert_map dropping half the experts
    (64, 1024, 384, 100, 8, 3, False),     # ragged: 12.5 rows per expert, K = 1024 / 384 (three K waves)
])
def test_moe_fused_producers_bit_identical(pkg, oracle_mod, dev, E, H, I, T, topk, fmt, mapped):
    """The grouped GEMMs with fused producers (quantization in w13, SwiGLU in w2), with and
    without the combine inside w2, give the same bits as the separate quantize / SwiGLU /
    combine launches; at T = 128 the layer is four launches (route, w13, w2, combine), three
    with the combine in w2; an expert_map's dropped routes contribute nothing."""
    ops = pkg.ops
    g = torch.Generator().manual_seed(E + T + H)
    Eg = 2 * E if mapped else E
    def wg(n, k):  # random codes: every packed FP6 pattern is a number
        return torch.randint(0, 256, (E, n, k * 3 // 4), generator=g, dtype=torch.uint8).to(dev)
    w13, w2 = wg(2 * I, H), wg(H, I)
    s13 = torch.randint(118, 124, (E, 2 * I, H // 32), generator=g, dtype=torch.uint8).to(dev)
    s2 = torch.randint(118, 124, (E, H, I // 32), generator=g, dtype=torch.uint8).to(dev)
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    wts, ids = torch.topk(torch.softmax(torch.randn(T, Eg, generator=g), -1), topk, -1)
    wts = (wts / wts.sum(-1, keepdim=True)).float().to(dev)
    ids = ids.int().to(dev)
    emap = None
    if mapped:
        gm = torch.full((Eg,), -1, dtype=torch.int32)
        gm[0::2] = torch.arange(E, dtype=torch.int32)
        emap = gm.to(dev)
    experts = pkg.Mxfp6Experts(fmt=fmt)
    e1, e2 = experts.process_weights_after_loading(w13, s13, w2, s2)
    routes = T * topk
    fused = (ops.grouped_fused_supported(routes, E, H, fmt), ops.grouped_fused_supported(routes, E, I, fmt))
    # the fused producers serve the 16-row-unit schedule (below 32 routed rows per expert)
    assert fused == ((routes < 32 * E),) * 2, fused
    out_f = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    before = dict(ops._COUNTS)
    experts.apply(out_f, x, e1, e2, wts, ids, "silu", Eg, emap, None, None, None, None, None, False)
    calls = {k: v - before.get(k, 0) for k, v in ops._COUNTS.items()
             if v != before.get(k, 0) and k != "workspace_miss"}  # launches, not allocations
    if (E, T) == (256, 128):
        assert fused[0] and calls == {"moe_route": 1, "grouped_gemm_quant": 1, "grouped_gemm_swiglu": 1,
                                      "moe_reduce": 1}, calls
    experts.fuse_combine = True  # the combine inside w2: three launches, the same bits
    out_c = torch.empty_like(out_f)
    before = dict(ops._COUNTS)
    experts.apply(out_c, x, e1, e2, wts, ids, "silu", Eg, emap, None, None, None, None, None, False)
    calls = {k: v - before.get(k, 0) for k, v in ops._COUNTS.items()
             if v != before.get(k, 0) and k != "workspace_miss"}  # launches, not allocations
    assert torch.equal(out_f, out_c)
    if (E, T) == (256, 128):
        assert calls == {"moe_route": 1, "grouped_gemm_quant": 1, "grouped_gemm_swiglu_combine": 1}, calls
    experts.fuse = False
    out_u = torch.empty_like(out_f)
    experts.apply(out_u, x, e1, e2, wts, ids, "silu", Eg, emap, None, None, None, None, None, False)
    assert torch.equal(out_f, out_u)
    experts.fuse_combine = False  # every stage its own launch
    out_s = torch.empty_like(out_f)
    experts.apply(out_s, x, e1, e2, wts, ids, "silu", Eg, emap, None, None, None, None, None, False)
    assert torch.equal(out_f, out_s)
    if mapped:  # tokens whose routes all left the node get exactly zero
        gone = (emap[ids.long()] < 0).all(dim=1)
        if gone.any():
            assert (out_f[gone] == 0).all()


@pytest.mark.parametrize("T,E,topk,bf16,renorm", [
    (1, 256, 8, False, True),
    (7, 4, 2, False, True),
    (128, 256, 8, False, True),    # c5 at T = 128: routing and the sort in one launch
    (128, 256, 8, True, True),     # bf16 logits: exact ties, to the lower expert
    (129, 256, 8, False, False),   # two chunks; weights over every expert
    (2048, 256, 8, False, True),   # c5 at T = 2048: routing with chunk histograms, then the scatter
    (2048, 256, 8, True, False),
    (3000, 64, 6, False, True),    # topk not dividing 1024: routing, then mxl_moe_route
    (100, 1024, 16, False, True),  # the widest expert count (16 logits per lane)
    (16, 1000, 64, True, True),    # the largest top-k; E not a multiple of 64
    (0, 256, 8, False, True),
])
def test_router_matches_oracle(pkg, oracle_mod, dev, T, E, topk, bf16, renorm):
    """softmax -> top-k -> renormalize -> token sort from router logits: ids (ties to the lower
    expert) and the sort tables bit-exact against the oracle; weights against the float64
    softmax within a few binary32 ulps."""
    g = torch.Generator().manual_seed(T + E + topk)
    logits = torch.randn(T, E, generator=g) * 2
    if bf16:
        logits = logits.bfloat16()
    w, ids, s, o, inv = torch.ops.mach_amd.moe_router(logits.to(dev), topk, renorm)
    rw, rids, rs, ro, rinv = oracle_mod.moe_router(logits.float().numpy(), topk, renorm)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(o.cpu().numpy(), ro)
    assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(inv.cpu().numpy(), rinv)
    if T:
        got = w.double().cpu().numpy()
        assert np.abs(got - rw).max() <= 4e-6 * np.abs(rw).max(), np.abs(got - rw).max()
        if bf16 and renorm:  # ties actually occurred among the selections
            srt = np.sort(logits.float().numpy(), axis=1)[:, ::-1]
            assert (srt[:, :topk + 1][:, 1:] == srt[:, :topk + 1][:, :-1]).any()


@pytest.mark.parametrize("T", [7, 128])
def test_moe_layer_from_router_logits(pkg, oracle_mod, dev, T):
    """The layer from logits (one router launch feeding the grouped GEMMs) equals
    select_experts + apply bit for bit, and the oracle's layer on the oracle's routing
    within the whole-layer bar; at c5 T = 128 it is three launches with the combine in w2
    (four by default, the same bits)."""
    E, H, I, topk = (256, 2048, 512, 8) if T == 128 else (4, 256, 128, 2)
    c13, s13, c2, s2, x, _, _ = _moe_case(oracle_mod, E, H, I, T, topk, 12035, 2)
    experts = pkg.Mxfp6Experts(fmt=2)
    w1, w2 = experts.process_weights_after_loading(
        torch.from_numpy(oracle_mod.pack_fp6(c13)).to(dev), torch.from_numpy(s13).to(dev),
        torch.from_numpy(oracle_mod.pack_fp6(c2)).to(dev), torch.from_numpy(s2).to(dev))
    logits = torch.randn(T, E, generator=torch.Generator().manual_seed(T)).to(dev)
    xd = x.to(dev)
    ops = pkg.ops
    experts.fuse_combine = True
    before = dict(ops._COUNTS)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    experts.apply_router(out, xd, w1, w2, logits, topk, True)
    calls = {k: v - before.get(k, 0) for k, v in ops._COUNTS.items()
             if v != before.get(k, 0) and k != "workspace_miss"}  # launches, not allocations
    if T == 128:  # three launches: router + sort, w13 + quantization, w2 + SwiGLU + combine
        assert calls == {"moe_router": 1, "grouped_gemm_quant": 1, "grouped_gemm_swiglu_combine": 1}, calls
    experts.fuse_combine = False
    out_d = torch.empty_like(out)
    experts.apply_router(out_d, xd, w1, w2, logits, topk, True)  # the default: four launches
    assert torch.equal(out, out_d)
    wts, ids = pkg.select_experts(logits, topk, True)
    out2 = torch.empty_like(out)
    experts.apply(out2, xd, w1, w2, wts, ids, "silu", E, None, None, None, None, None, None, False)
    assert torch.equal(out, out2)
    rw, rids, *_ = oracle_mod.moe_router(logits.cpu().numpy(), topk, True)
    ref = oracle_mod.bf16_to_f32(oracle_mod.moe_ref(x, c13, s13, c2, s2, rw.astype(np.float32), rids, 2))
    got = out.float().cpu().numpy()
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-2


@pytest.mark.parametrize("E,N,K,T,topk,swiglu,fmt,drop", [
    (256, 2048, 512, 128, 8, True, 2, False),    # c5 T = 128 down projection: 16-row units + SwiGLU
    (256, 2048, 512, 128, 8, False, 2, False),   # the same on MXFP8 operands
    (8, 256, 384, 40, 4, True, 3, True),         # E3M2, dropped routes and fully dropped tokens
    (16, 264, 512, 60, 6, False, 0, True),       # E4M3, ragged N, dropped routes
    (32, 512, 256, 20, 16, True, 2, False),      # the largest top-k
])
def test_grouped_combine_matches_reduce(pkg, oracle_mod, dev, E, N, K, T, topk, swiglu, fmt, drop):
    """The down projection with the weighted combine in its launch writes the bits of the
    grouped GEMM followed by moe_reduce: twice in a row (the second call with fewer tokens,
    so the per-token counters must have been left zero) and under graph replay."""
    ops = pkg.ops
    g = torch.Generator().manual_seed(E + N + K + T)
    ids = torch.randint(0, E, (T, topk), generator=g, dtype=torch.int32)
    if drop:  # ids outside [0, E) are dropped by the sort; tokens 0-2 lose every route
        ids[::3, 1] = E + 3
        ids[:3] = -1
    wts = torch.rand(T, topk, generator=g).float()
    wts = wts / wts.sum(-1, keepdim=True)
    w = torch.randint(0, 256, (E, N, K if fmt == 0 else K * 3 // 4), generator=g, dtype=torch.uint8)
    if fmt == 0:  # E4M3 codes without the NaN pattern (every FP6 pattern is a number)
        w[(w & 0x7F) == 0x7F] = 0x3F
    w = w.to(dev)
    s = torch.randint(118, 124, (E, N, K // 32), generator=g, dtype=torch.uint8).to(dev)
    w_t, s_t = ops.pack_weight(w, s, fmt)
    R = T * topk
    assert ops.grouped_combine_supported(R, E, N, K, fmt, swiglu, topk)
    # 96-row units (tens of rows per expert) keep the combine in its own launch
    assert not ops.grouped_combine_supported(64 * E, E, N, K, fmt, swiglu, topk)

    def case(Tc):
        idc = ids[:Tc].to(dev)
        routes, offsets, inverse = torch.ops.mach_amd.moe_route(idc, E)
        Rc = Tc * topk
        if swiglu:
            gu = (torch.randn(Rc, 2 * K, generator=g) * 2).bfloat16().to(dev)
            y = torch.ops.mach_amd.grouped_gemm_swiglu(gu, offsets, Rc, w_t, s_t, N, K, fmt, ops.CEIL_DIV448)
        else:
            a, sa = torch.ops.mach_amd.quantize_mxfp8((torch.randn(Rc, K, generator=g)).bfloat16().to(dev), 0)
            y = torch.ops.mach_amd.grouped_gemm(a, sa, None, 1, offsets, Rc, w_t, s_t, N, K, fmt)
        ref = torch.empty(Tc, N, dtype=torch.bfloat16, device=dev)
        wd = wts[:Tc].to(dev)
        torch.ops.mach_amd.moe_reduce(ref, y, wd, inverse)

        def run(out):
            if swiglu:
                torch.ops.mach_amd.grouped_gemm_swiglu_combine(out, gu, offsets, Rc, w_t, s_t, N, K, fmt,
                                                               ops.CEIL_DIV448, routes, inverse, wd)
            else:
                torch.ops.mach_amd.grouped_gemm_combine(out, a, sa, None, 1, offsets, Rc, w_t, s_t, N, K, fmt,
                                                        routes, inverse, wd)
        return ref, run

    ref, run = case(T)
    out = torch.full((T, N), float("nan"), dtype=torch.bfloat16, device=dev)
    run(out)
    assert torch.equal(out, ref)
    if drop:
        assert (out[:3] == 0).all()
    ref2, run2 = case(T // 2 + 1)
    out2 = torch.empty_like(ref2)
    run2(out2)
    assert torch.equal(out2, ref2)
    # graph replays with eager calls between them: the counters stay consistent
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run(out)
        graph = torch.cuda.CUDAGraph()
        out_g = torch.empty_like(ref)
        with torch.cuda.graph(graph, stream=stream):
            run(out_g)
        for _ in range(3):
            out_g.zero_()
            graph.replay()
            stream.synchronize()
            assert torch.equal(out_g, ref)
            run(out)
            stream.synchronize()
            assert torch.equal(out, ref)
    torch.cuda.current_stream().wait_stream(stream)
