"""GPU parity of the wide-tile prefill GEMM (128-row workgroup tiles, K-stage ring,
optional K splits) against the oracle, on the shapes that exercise its edges:
ragged M and N, a K that ends in half a 512-wide super-tile, forced split counts,
more tiles than CUs (whole-K rounds plus a K-split remainder),
every weight format, bias, block-FP8 scales, and grouped experts with skewed,
empty and multi-block row ranges.  Same bar as the other GEMM tests."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import _act, _check, _weights

pytestmark = pytest.mark.gpu


def force(monkeypatch, ops, cfg=None, **changes):
    """Pin the kernel selection for this test (``ops._tuning``), merged with any pin already
    set: ``cfg`` is a wide-tile spec "NT,S" or "NT,1,h"; keywords set other fields."""
    cur = ops._tuning
    f = {k: getattr(cur, k) for k in ("kernel", "splits", "tile_n", "tile_m", "hybrid", "waves")} \
        if cur is not None else {"kernel": -1, "splits": 0, "tile_n": 0, "tile_m": 0, "hybrid": 0, "waves": 0}
    if cfg:
        parts = cfg.split(",")
        f.update(tile_n=int(parts[0]), splits=int(parts[1]), hybrid=int(len(parts) > 2 and parts[2] == "h"))
    f.update(changes)
    monkeypatch.setattr(ops, "_tuning", pkg_options(ops, **f))


def pkg_options(ops, kernel, splits, tile_n, tile_m, hybrid, waves=0):
    from vllm_mach_amd import _lib
    return _lib.GemmOptions(0, kernel, splits, tile_n, tile_m, hybrid, waves)


@pytest.mark.parametrize("M,N,K,fmt,cfg,bias", [
    (64, 256, 512, 0, None, False),
    (200, 1000, 768, 0, "2,1", True),     # K = 1.5 super-tiles, ragged M
    (300, 640, 2304, 2, "2,3", False),    # 3 K splits over 4.5 super-tiles
    (130, 384, 1280, 3, "1,2", False),
    (512, 512, 1792, 0, "1,4", True),
    (257, 136, 1280, 2, None, False),     # N not a multiple of 16
    (96, 2048, 4096, 0, "2,8", False),
    (384, 1024, 2560, 0, "4,2", True),    # 3-slot ring, ragged K split
    (130, 1280, 768, 2, "4,1", False),
    (256, 700, 1280, 3, "4,3", False),    # N not a multiple of 256
])
def test_wide_mx_gemm(pkg, oracle_mod, dev, monkeypatch, M, N, K, fmt, cfg, bias):
    ops = pkg.ops
    if cfg:
        force(monkeypatch, ops, cfg)
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 11 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 7 + M)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(3)) * 0.5).bfloat16() if bias else None
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, b.to(dev) if bias else None)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
    if bias:
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref + b.float().numpy()[None, :]))
    _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,fmt,cfg,bias", [
    (200, 1000, 768, 0, "2,1", True),      # ragged M, K = 1.5 super-tiles
    (300, 640, 2304, 2, "2,3", False),     # 3 K splits over 4.5 super-tiles
    (130, 384, 1280, 3, "1,2", False),     # one n-tile per group: both waves copy its scales
    (384, 1024, 2560, 0, "4,2", True),     # 3-slot ring
    (256, 700, 1280, 3, "4,3", False),     # N not a multiple of 256
    (512, 8320, 1024, 0, "2,1,h", True),   # hybrid: whole-K rounds then the split remainder
    (512, 2560, 9216, 0, "2,3", False),    # c2 M = 512
    (256, 17408, 5120, 2, "2,1,h", False), # c4 M = 256
])
def test_wide_eight_waves(pkg, oracle_mod, dev, monkeypatch, M, N, K, fmt, cfg, bias):
    """Eight waves per workgroup (two per SIMD, each half the tile's rows): bit-identical to
    the four-wave kernel (the same MFMA chain per 16 x 16 output tile) and within the bar."""
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 13 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 5 + M)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(6)) * 0.5).bfloat16().to(dev) if bias else None
    force(monkeypatch, ops, cfg, waves=4)
    y4 = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, b)
    force(monkeypatch, ops, cfg, waves=8)
    y8 = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, b)
    assert torch.equal(y8, y4)
    assert torch.equal(torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, b), y8)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
    if bias:
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref + b.float().cpu().numpy()[None, :]))
    _check(y8.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,fmt,same_as", [
    (512, 2560, 9216, 0, "2,3"),       # c2 M = 512
    (128, 17408, 5120, 2, "2,1"),      # c4 M = 128
    (256, 17408, 5120, 2, "2,1,h"),    # c4 M = 256: whole-K round plus split remainder
])
def test_wide_mx_auto_plan(pkg, oracle_mod, dev, monkeypatch, M, N, K, fmt, same_as):
    """The planner's own MX choice on 128 x 128 tiles (eight waves): bit-identical to the
    four-wave kernel on the same tiles and splits."""
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 29 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 17 + M)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    monkeypatch.setattr(ops, "_tuning", None)
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    force(monkeypatch, ops, same_as, waves=4)
    y4 = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, None)
    assert torch.equal(y, y4)


@pytest.mark.parametrize("M,N,K,cfg", [
    (64, 256, 512, None),
    (200, 384, 1280, "2,2"),
    (300, 1024, 768, "1,1"),
    (200, 1024, 1280, "4,2"),
    (512, 18432, 2560, None),
])
def test_wide_block_fp8_gemm(pkg, oracle_mod, dev, monkeypatch, M, N, K, cfg):
    ops = pkg.ops
    if cfg:
        force(monkeypatch, ops, cfg)
    g = torch.Generator().manual_seed(91 + M + K)
    w = torch.randn(N, K, generator=g) * 0.02
    wb = w.reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    x = torch.randn(M, K, generator=g).bfloat16()
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    y = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    rq, rs = oracle_mod.quant_block_fp8(x)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), rq)
    ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
    _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,cfg", [
    (200, 1024, 1280, "2,2"),
    (512, 18432, 2560, "2,1"),
    (128, 18432, 2560, "1,3"),
    (300, 640, 768, "2,1,h"),
])
def test_wide_block_fp8_eight_waves(pkg, oracle_mod, dev, monkeypatch, M, N, K, cfg):
    """Block-FP8 with eight waves (two per SIMD, one's per-K128 folds under the other's
    MFMAs): bit-identical to the four-wave kernel (each 16 x 16 output tile sees the same
    MFMA chain and folds) and within the bar of the oracle."""
    ops = pkg.ops
    g = torch.Generator().manual_seed(191 + M + K)
    w = torch.randn(N, K, generator=g) * 0.02
    wb = w.reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    x = torch.randn(M, K, generator=g).bfloat16()
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    force(monkeypatch, ops, cfg, waves=4)
    y4 = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    force(monkeypatch, ops, cfg, waves=8)
    y8 = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    assert torch.equal(y8, y4)
    if N * K <= 4_000_000:
        rq, rs = oracle_mod.quant_block_fp8(x)
        ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
        _check(y8.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,same_as", [
    (64, 1024, 1280, None),            # half the 128-row tile past the last row
    (200, 2048, 1536, None),           # ragged M
    (256, 18432, 2560, "2,1,h"),       # c3: 288 tiles, whole-K round plus split remainder
    (512, 18432, 2560, "2,1"),         # c3: three whole-K rounds
])
def test_wide_block_fp8_auto_plan(pkg, oracle_mod, dev, monkeypatch, M, N, K, same_as):
    """The planner's own block-FP8 choice (eight waves on 128 x 128 tiles): within the bar of
    the oracle, and at the c3 shapes bit-identical to the four-wave kernel on the same tiles."""
    ops = pkg.ops
    g = torch.Generator().manual_seed(401 + M + N)
    w = torch.randn(N, K, generator=g) * 0.02
    wb = w.reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    x = torch.randn(M, K, generator=g).bfloat16()
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    monkeypatch.setattr(ops, "_tuning", None)
    y = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    if same_as:
        force(monkeypatch, ops, same_as, waves=4)
        y4 = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
        assert torch.equal(y, y4)
    else:
        rq, rs = oracle_mod.quant_block_fp8(x)
        ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
        _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,fmt,cfg,bias", [
    (512, 8320, 1024, 0, "2,1,h", True),     # 260 tiles: 256 whole-K, 4 split two ways
    (300, 11000, 1536, 2, "2,1,h", False),   # ragged M and N: 258 tiles, remainder split three ways
    (512, 4160, 1280, 3, "1,1,h", True),     # 64-wide tiles, K = 2.5 super-tiles
    (512, 16640, 1024, 0, "4,1,h", False),   # 3-slot ring: 260 tiles of 128 x 256
])
def test_wide_hybrid_mx_gemm(pkg, oracle_mod, dev, monkeypatch, M, N, K, fmt, cfg, bias):
    """More tiles than CUs: full rounds of whole-K tiles write bf16, the remainder is split
    in K into compact partials and summed by the tile reduce; repeated calls agree."""
    ops = pkg.ops
    force(monkeypatch, ops, cfg)
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 5 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 9 + M)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(4)) * 0.5).bfloat16() if bias else None
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, b.to(dev) if bias else None)
    assert torch.equal(torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, b.to(dev) if bias else None), y)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
    if bias:
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref + b.float().numpy()[None, :]))
    _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,cfg", [(512, 8320, 1280, "2,1,h"), (512, 16640, 1024, "4,1,h")])
def test_wide_hybrid_block_fp8_gemm(pkg, oracle_mod, dev, monkeypatch, M, N, K, cfg):
    ops = pkg.ops
    force(monkeypatch, ops, cfg)
    g = torch.Generator().manual_seed(33 + K)
    wb = (torch.randn(N, K, generator=g) * 0.02).reshape(N // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(N, K).to(torch.float8_e4m3fn)
    x = torch.randn(M, K, generator=g).bfloat16()
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    y = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, None)
    rq, rs = oracle_mod.quant_block_fp8(x)
    ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
    _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,fmt,cfg,bias", [
    (64, 256, 512, 0, None, False),
    (200, 1000, 768, 0, "2,1", True),      # K = 1.5 super-tiles, ragged M
    (100, 640, 2304, 2, "2,3", False),     # 3 K splits over 4.5 super-tiles
    (257, 136, 1280, 3, "2,1", True),      # N not a multiple of 16
    (130, 1024, 2560, 0, "4,2", True),     # 3-slot ring, ragged K split
    (190, 700, 1280, 2, "4,1", False),     # N not a multiple of 256
    (300, 8320, 1024, 0, "2,1,h", True),   # 5 x 65 = 325 tiles: hybrid with 69 split tiles
    (130, 16640, 1024, 3, "4,1,h", False),  # 3 x 65 = 195 < 256 tiles: the plain launch
])
def test_wide_mx_gemm_64_row_tiles(pkg, oracle_mod, dev, monkeypatch, M, N, K, fmt, cfg, bias):
    """The 64-row workgroup tile (four m-tiles, one activation-scale wave) on the edge
    shapes of the 128-row tests."""
    force(monkeypatch, pkg.ops, tile_m=4)
    test_wide_mx_gemm(pkg, oracle_mod, dev, monkeypatch, M, N, K, fmt, cfg, bias)


@pytest.mark.parametrize("M,N,K,cfg", [(100, 384, 1280, "2,2"), (200, 1024, 1280, "4,1"), (300, 8320, 1280, "2,1,h")])
def test_wide_block_fp8_64_row_tiles(pkg, oracle_mod, dev, monkeypatch, M, N, K, cfg):
    force(monkeypatch, pkg.ops, tile_m=4)
    test_wide_block_fp8_gemm(pkg, oracle_mod, dev, monkeypatch, M, N, K, cfg)


@pytest.mark.parametrize("mt", [None, "4", "8"])
@pytest.mark.parametrize("fmt", [0, 2])
@pytest.mark.parametrize("T", [400, 340])
def test_wide_grouped_gemm_skewed_experts(pkg, oracle_mod, dev, monkeypatch, fmt, mt, T):
    """Expert 0 takes 300 routes (three 128-row blocks, the last of 44 rows on the 64-row
    path, or five 64-row blocks), expert 1 none, the rest about 83 (T = 400) or 63 (T =
    340) each, so 128-row blocks of both paths meet in one launch; rows are gathered
    through the sorted route list (row_div = topk)."""
    ops = pkg.ops
    if mt:
        force(monkeypatch, ops, tile_m=int(mt))
    E, N, K, topk = 8, 384, 1024, 2
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(2, E, (T, topk), generator=g, dtype=torch.int32)
    ids[:300, 0] = 0
    parts = [_weights(oracle_mod, N, K, fmt, 0.02, 40 + e) for e in range(E)]
    stored = np.stack([p[2] for p in parts])
    scales = np.stack([p[1] for p in parts])
    w_t, s_t = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(scales).to(dev), fmt)
    x = _act(T, K, 77)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    routes, offsets, _ = torch.ops.mach_amd.moe_route(ids.to(dev), E)
    R = T * topk
    assert R >= 32 * E  # the wide grouped kernel serves this shape
    y = torch.ops.mach_amd.grouped_gemm(a, sa, routes, topk, offsets, R, w_t, s_t, N, K, fmt)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    off = offsets.cpu().numpy()
    rt = routes.cpu().numpy()
    got = y.float().cpu().numpy()
    assert off[1] - off[0] == 300 and off[2] == off[1]
    for e in range(E):
        lo, hi = int(off[e]), int(off[e + 1])
        if lo == hi:
            continue
        rows = rt[lo:hi] // topk
        ref = oracle_mod.mx_gemm_ref(rc[rows], rs[rows], parts[e][0], parts[e][1], fmt)
        _check(got[lo:hi], oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref)))


def test_wide_grouped_gemm_max_experts(pkg, oracle_mod, dev, monkeypatch):
    """The most experts the grouped wide kernel takes (1024: its expert prefix shares the
    LDS with the second workgroup on each CU), about 32 routed rows per expert, forced onto
    the wide kernel: within the bar of the 96-row streaming schedule on every route and of
    the oracle on the first, the last and the largest expert."""
    ops = pkg.ops
    E, N, K, T, topk, fmt = 1024, 256, 512, 4096, 8, 2
    g = torch.Generator().manual_seed(2024)
    ids = torch.randint(0, E, (T, topk), generator=g, dtype=torch.int32)
    packed = torch.randint(0, 256, (E, N, K * 3 // 4), generator=g, dtype=torch.uint8)  # every FP6 pattern is a number
    scales = torch.randint(118, 124, (E, N, K // 32), generator=g, dtype=torch.uint8)
    w_t, s_t = ops.pack_weight(packed.to(dev), scales.to(dev), fmt)
    routes, offsets, _ = torch.ops.mach_amd.moe_route(ids.to(dev), E)
    R = T * topk
    x = _act(T, K, 31)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    force(monkeypatch, ops, kernel=ops.KERNEL_WIDE)
    y = torch.ops.mach_amd.grouped_gemm(a, sa, routes, topk, offsets, R, w_t, s_t, N, K, fmt)
    force(monkeypatch, ops, kernel=ops.KERNEL_STREAM_WIDE)
    y_s = torch.ops.mach_amd.grouped_gemm(a, sa, routes, topk, offsets, R, w_t, s_t, N, K, fmt)
    got = y.float().cpu().numpy()
    _check(got, y_s.float().cpu().numpy())
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    off, rt = offsets.cpu().numpy(), routes.cpu().numpy()
    for e in sorted({0, E - 1, int(np.argmax(off[1:] - off[:-1]))}):
        lo, hi = int(off[e]), int(off[e + 1])
        if lo == hi:
            continue
        rows = rt[lo:hi] // topk
        ref = oracle_mod.mx_gemm_ref(rc[rows], rs[rows], oracle_mod.unpack_fp6(packed[e].numpy()),
                                     scales[e].numpy(), fmt)
        _check(got[lo:hi], oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref)))


@pytest.mark.parametrize("M,N,K,fmt", [
    (1, 2560, 9216, 0),      # sixteen single-buffered waves
    (16, 2560, 9216, 0),
    (7, 17408, 5120, 2),     # persistent workgroups with 4 and 5 n-tiles (double-buffered pairs)
    (3, 200, 384, 3),        # ragged N, three K128 slices over eight waves
    (16, 4096, 10240, 0),
    (16, 1000, 128, 2),      # a single slice
    (16, 2048, 2048, 0),     # c1's shape: 128 n-tiles, four super-tiles
    (5, 18408, 2560, 3),     # 1151 n-tiles, the last 8 columns wide
])
def test_stream_decode_gemm(pkg, oracle_mod, dev, M, N, K, fmt):
    """The weight-streaming decode kernel (M <= 16) against the oracle."""
    ops = pkg.ops
    wc, ws, stored = _weights(oracle_mod, N, K, fmt, 0.02, 13 + N + K)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), fmt)
    x = _act(M, K, 3 + M)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    rc, rs = oracle_mod.quant_mxfp8(x, 0)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(9)) * 0.5).bfloat16()
    y = torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, fmt, b.to(dev))
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, fmt)))
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref + b.float().numpy()[None, :]))
    _check(y.float().cpu().numpy(), ref)


def test_wide_split_repeat_and_replay(pkg, oracle_mod, dev, monkeypatch):
    """K splits: repeated calls and graph replays (with eager calls between them) give
    the same bits, since the partials are summed in split order."""
    ops = pkg.ops
    M, N, K = 300, 1024, 2304
    force(monkeypatch, ops, "2,3")
    wc, ws, stored = _weights(oracle_mod, N, K, 0, 0.02, 17)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(stored).to(dev), torch.from_numpy(ws).to(dev), 0)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(_act(M, K, 5).to(dev), 0)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(2)) * 0.5).bfloat16().to(dev)

    def run():
        return torch.ops.mach_amd.mx_gemm(a, sa, tiled, tiled_s, N, K, 0, b)

    first = run()
    for _ in range(3):
        assert torch.equal(run(), first)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = run()
        for _ in range(3):
            graph.replay()
            stream.synchronize()
            assert torch.equal(out, first)
            assert torch.equal(run(), first)  # eager between replays
    torch.cuda.current_stream().wait_stream(stream)
    rc, rs = oracle_mod.quant_mxfp8(_act(M, K, 5), 0)
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(oracle_mod.mx_gemm_ref(rc, rs, wc, ws, 0)))
    ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref + b.float().cpu().numpy()[None, :]))
    _check(first.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,bias", [
    (1, 18432, 2560, False),   # c3's shape: five waves, double-buffered n-tiles
    (5, 200, 384, True),       # ragged N, three slices in one super-tile
    (16, 1024, 5120, False),   # ten super-tiles: two per wave
    (3, 512, 8192, True),      # the largest K of the streamed block-FP8 path
    (16, 2560, 9216, False),   # past it: the generic kernel
])
def test_stream_block_fp8_gemm(pkg, oracle_mod, dev, M, N, K, bias):
    """Block-FP8 at decode sizes on the weight-streaming kernel (raw MFMA per K128
    slice folded with the fp32 activation and weight block scales)."""
    ops = pkg.ops
    g = torch.Generator().manual_seed(7 * M + K)
    Np = (N + 127) // 128 * 128
    wb = (torch.randn(Np, K, generator=g) * 0.02).reshape(Np // 128, 128, K // 128, 128)
    sb = (wb.abs().amax(dim=(1, 3)) / 448.0).float()
    wq = (wb / sb[:, None, :, None]).reshape(Np, K).to(torch.float8_e4m3fn)[:N].contiguous()
    x = torch.randn(M, K, generator=g).bfloat16()
    b = (torch.randn(N, generator=g) * 0.5).bfloat16() if bias else None
    tiled, _ = ops.pack_weight(wq.to(dev), None, 0)
    q, s = torch.ops.mach_amd.quantize_block_fp8(x.to(dev))
    y = torch.ops.mach_amd.block_fp8_gemm(q, s, tiled, sb.to(dev), N, K, b.to(dev) if bias else None)
    rq, rs = oracle_mod.quant_block_fp8(x)
    ref = oracle_mod.bf16_to_f32(oracle_mod.block_fp8_gemm_ref(rq, rs, wq.view(torch.uint8).numpy(), sb.numpy()))
    if bias:
        ref = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(ref + b.float().numpy()[None, :]))
    _check(y.float().cpu().numpy(), ref)


@pytest.mark.parametrize("M,N,K,cfg,f16,alpha,bias", [
    (200, 1000, 2560, "2,3", 1, 0.375, False),   # ragged M and N: partial tiles in both
    (256, 1000, 2560, "1,4", 0, 0.5, True),      # 64-column tiles, bias after the scaled rounding
    (512, 8320, 1024, "2,1,h", 1, 0.375, True),  # hybrid: 260 tiles, whole-K round plus split units
    (130, 640, 2048, "4,2", 1, 0.5, False),      # 256-column tiles, three-slot ring
])
def test_wide_split_epilogue_rounds_once(pkg, oracle_mod, dev, M, N, K, cfg, f16, alpha, bias):
    """The wide kernel's K split (fragment-ordered partials summed by the tile reduce) with
    the output scale, format and bias, through the C ABI: integer operands make every sum
    exact, so the output must equal round(alpha * exact) (then + bias, rounded again) bit for
    bit in bf16 or fp16 -- rows and columns past M and N included in the tiles, not stored."""
    from test_gpu_boundary_ops import _integer_operands
    from vllm_mach_amd import _lib
    ops = pkg.ops
    x, wp, ws, exact = _integer_operands(oracle_mod, M, N, K, 900 + M + N)
    tiled, tiled_s = ops.pack_weight(torch.from_numpy(wp).to(dev), torch.from_numpy(ws).to(dev), 3)
    a, sa = torch.ops.mach_amd.quantize_mxfp8(x.to(dev), 0)
    parts = cfg.split(",")
    opts = _lib.GemmOptions(0, 1, int(parts[1]), int(parts[0]), 0, int(len(parts) > 2), 4, f16, alpha)
    need = _lib.query("mxl_gemm_workspace_bytes_ex", M, N, K, 3, 0, _lib.options_ptr(opts))
    assert need > 0  # the configuration splits K
    ws_buf = torch.empty(need, dtype=torch.uint8, device=dev)
    dtype = torch.float16 if f16 else torch.bfloat16
    # the bias is bf16 whatever the output format (mxl_gemm_options: added in binary32 after
    # the scaled rounding, then rounded again)
    b = (torch.randint(-64, 64, (N,), generator=torch.Generator().manual_seed(3)).float() / 4).bfloat16()
    bd = b.to(dev)
    out = torch.full((M, N + 8), 7.0, dtype=dtype, device=dev)  # ldc > N: the pad stays untouched
    _lib.call("mxl_mx_gemm_ex", a.data_ptr(), sa.data_ptr(), M, tiled.data_ptr(), tiled_s.data_ptr(), N, K, 3,
              bd.data_ptr() if bias else None, out.data_ptr(), N + 8, ws_buf.data_ptr(), need,
              _lib.options_ptr(opts), torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize(dev)
    expected = torch.from_numpy(exact.astype(np.float32) * np.float32(alpha)).to(dtype)
    if bias:
        expected = (expected.float() + b.float()[None, :]).to(dtype)
    got = out.cpu()
    assert torch.equal(got[:, :N], expected)
    assert torch.all(got[:, N:] == 7.0)
